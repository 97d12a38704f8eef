// paged_prefill_dma.hip - chunked / paged prefill attention on gfx950, with the K/V pages streamed into LDS by
// asynchronous global->LDS loads (16-bit caches, and 8-bit int8 / fp8 e4m3 codes).
//
// Replaces the reference's prefill branch of kernels::attention (flash_attn_wmma_kernel,
// src/kernels/attention.cu:22-286, dispatched at :460-474 and routed from src/model/qwen_model.cu:147-151), which
// attends only to the chunk's own contiguous K/V with a causal mask (key n > query m masked, :173-174), and extends
// it to queries over a cached prefix: query token t of row b at position ctx[b] + t attends keys 0 .. ctx[b] + t
// read from the paged cache (prefix and chunk, after the chunk's append).  Without a block table the keys are the
// chunk's contiguous [B, S, Hkv, D] tensors and ctx = 0: exactly the reference's causal prefill.  With S = 1 it is
// the decode attention.
//
// Mapping: a workgroup serves 128 query rows of one (row b, kv head); a query row is a (token, head-in-group) pair,
// so the GQA heads of a kv head share every K/V page.  Each wave owns 16 query rows per row group as the 16
// columns of its MFMA tiles: S^T[key, row] = K Q^T with K (16 keys x 32 dims) as the A operand from LDS and Q^T in
// registers, an online softmax per column (causal limit per column) over a step of pages, and O^T += V^T P^T as
// 16x16x32 products over 32 keys with P^T straight from the score registers.
//
// Pages reach LDS without passing through registers: every 16-byte chunk of a step's K and V pages goes from HBM
// straight into LDS with global_load_lds_dwordx4 (each lane's 16 bytes land at the instruction's LDS base +
// 16 * lane), with no staging registers.  NS stages rotate (two at head_dim 128
// and 256, three at 64): step i + NS - 1 is requested as soon as every wave has finished step i - 1, so NS - 1
// steps of loads are in flight behind the step being computed, with one barrier per step.  Each stage is its own LDS object and the main loop is unrolled by NS, so the compiler can tell
// which stage a load writes and does not hold the compute of one stage behind the loads into another.
//
// At head_dim <= 128 a workgroup is four waves of 32 query rows (two row groups of 16 MFMA columns): every K and
// V^T operand read from LDS feeds two matrix products, which halves the LDS reads and the per-step scalar work per
// query row.  Within a step the scores' products go out first; the scalar address work of the next step's loads
// (block-table reads, page offsets) then runs while they execute instead of ahead of them.
//
// Both tiles stay row-major (key-major).  The K operand of S^T = K Q^T reads 8 consecutive dims of one key;
// the V^T operand of O^T += V^T P^T needs 8 consecutive keys of one dim, which ds_read_b64_tr_b16 gives
// directly: within each 16-lane group, lane 4r + q supplies the address of dims 4q .. 4q + 3 of key row r, and
// lane j receives dim j of rows 0..3.  16-byte chunks of a key row are XOR-swizzled by row so that neither the
// K reads (16 rows, one chunk) nor the transposed V reads (4 rows, two chunks per 16-lane group) collide in LDS
// banks; the loads apply the same swizzle by choosing which chunk each lane fetches.
//
// 8-bit caches load their codes the same way (half the bytes per page) and convert them when an operand is read:
// the K operand is an 8-byte read of 8 codes, the V^T operand one ds_read_b64_tr_b8 (within each 16-lane group,
// lanes 2r and 2r + 1 supply the two halves of key row r's 16 dims, and lane j receives dim j of rows 0..7,
// which are the 8 keys of one k-slot group), both turned into 8 MFMA-type values by the gfx950 conversions.
// Under a bf16 q the score products are bf16 (q whole), and the PV products f16: the codes are exact in both
// types, and f16's 11 bits hold P in one product where bf16 P needs a hi + lo pair (C4-shaped prefill: fp8 300 ->
// 240 us, int8 356 -> 333 us).  int8 per-token scales (fp32 [N, 16, Hkv]) travel with their page into the stage
// by 4-byte loads; fp8 per-head scales fold into the score scale and the output.
//
// Two kinds of pages are converted in LDS instead, each wave converting the runs it loaded, in place, after its
// own wait for them and before the barrier that publishes the step (no barrier of its own): bf16 pages' V tiles
// to f16, so that their PV products take f16 P in one product (a V value beyond f16's range reruns the
// workgroup on bf16 products), and int8 pages at head_dim <= 128 to 16-bit f16 tiles read as an f16 cache's.
//
// Keys past the row's end and keys on invalid pages are fetched from a zero block instead, so masked keys meet
// zero V rows (their probabilities are exactly zero) and no lane reads outside the cache.
#include "mfma_common.h"

namespace ffkv
{

namespace
{

constexpr int kDmaRows = 128;  // query rows per workgroup: 8 waves x 16 rows (RG = 1) or 4 waves x 32 rows (RG = 2)
// LDS stages of the load pipeline (steps in flight behind the computed one, + 1).  At head_dim 128 a step is four
// pages (64 keys) and two stages hold as many bytes in flight as three of two pages, with half the per-step
// scalar work, barriers and row reductions per key (C4-shaped prefill: bf16 320 -> 293 us, int8 401 -> 366 us);
// head_dim 256 (two pages per step) is also faster with two (718 -> 689 us), head_dim 64 is even.
#ifndef FFKV_PREFILL_STAGES
#define FFKV_PREFILL_STAGES 2  // head_dim 128 and 256
#endif
#ifndef FFKV_PREFILL_STAGES64
#define FFKV_PREFILL_STAGES64 3
#endif
template <int D>
constexpr int kDmaStages = D == 64 ? FFKV_PREFILL_STAGES64 : FFKV_PREFILL_STAGES;
static_assert(kDmaStages<64> >= 2 && kDmaStages<64> <= 4 && kDmaStages<128> >= 2 && kDmaStages<128> <= 4,
              "two to four stages");
constexpr int kXcds = 8;  // MI355X: workgroups are dealt to 8 XCDs (separate L2s) in turn

#ifndef FFKV_PREFILL_XCD
#define FFKV_PREFILL_XCD 1
#endif

#ifndef FFKV_PREFILL_VCONV
#define FFKV_PREFILL_VCONV 1  // bf16 pages: V tiles converted to f16 in LDS by the waves that load them
#endif
#ifndef FFKV_PREFILL_AHEAD
#define FFKV_PREFILL_AHEAD 1  // with three or more stages: tiles converted in LDS one step ahead, behind the scores
#endif
#ifndef FFKV_PREFILL_L_MFMA
#define FFKV_PREFILL_L_MFMA 1  // fp8 pages: the denominator of f16 P by a product with a tile of ones
#endif
#ifndef FFKV_PREFILL_C16
#define FFKV_PREFILL_C16 1  // int8 pages at head_dim <= 128: tiles converted to f16 in LDS by the waves that load them
#endif
#ifndef FFKV_PREFILL_I8_BF
#define FFKV_PREFILL_I8_BF 0  // int8 with bf16 q: bf16 score products (1) or f16 ones with q converted whole (0)
#endif

#ifndef FFKV_PREFILL_RG
#define FFKV_PREFILL_RG 2  // row groups of 16 query rows per wave at head_dim <= 128
#endif

#ifndef FFKV_PREFILL_RG256
#define FFKV_PREFILL_RG256 1  // the same at head_dim 256 (two take 512 registers, one wave per SIMD: 287 -> 908 us)
#endif

#ifndef FFKV_PREFILL_DMA_KP64
#define FFKV_PREFILL_DMA_KP64 4  // pages per step at head_dim 64
#endif

#ifndef FFKV_PREFILL_DMA_KP128
#define FFKV_PREFILL_DMA_KP128 4  // pages per step at head_dim 128
#endif

#ifndef FFKV_PREFILL_DMA_KP256
#define FFKV_PREFILL_DMA_KP256 4  // pages per step at head_dim 256 (the shared-prefix partials take 2)
#endif

#ifndef FFKV_PREFILL_V16
#define FFKV_PREFILL_V16 1  // PV products in f16 for 8-bit caches whose score products are bf16
#endif

#define FFKV_LDS __attribute__((address_space(3)))

using i32x2 = int __attribute__((ext_vector_type(2)));
#define FFKV_CONST __attribute__((address_space(4)))  // read-only for the kernel's lifetime: scalar loads

// Source of the chunks of keys that are not loaded: 64 lanes x 16 bytes of zeros (never written).
__device__ __align__(16) uint32_t g_zero_chunks[256];

// EB: bytes per cached element (2, or 1 for int8 / fp8 codes); SC: int8 scales; W: waves per workgroup; PFX:
// shared-prefix partials, whose head_dim 256 f16 variant spills registers at 4 pages per step
template <int D, int EB, bool SC, int W, bool PFX>
struct DmaCfg
{
    static constexpr int KP = D == 64 ? FFKV_PREFILL_DMA_KP64
                                      : (D == 128 ? FFKV_PREFILL_DMA_KP128 : (PFX ? 2 : FFKV_PREFILL_DMA_KP256));
    static constexpr int RB = D * EB;                  // bytes of one key row (one kv head)
    static constexpr int CPT = RB / 16;                // 16-byte chunks per key row
    static constexpr int CHUNKS = kBlockSize * CPT;    // chunks per page
    static constexpr int TILEB = KP * kBlockSize * RB; // bytes of a step's K (or V) tile
    static constexpr int SCB = SC ? 2 * KP * kBlockSize * 4 : 0;  // int8 scales of the step: K then V
    static constexpr int IPR = KP * CHUNKS / 64;       // 64-chunk load runs per tile
    static constexpr int RPW = 2 * IPR / W;            // runs per wave and step (K runs first, then V)
    static_assert(RPW >= 1 && (2 * IPR) % W == 0, "every wave loads whole 64-chunk runs");
    static_assert(CHUNKS % 64 == 0, "a 64-chunk run stays inside one page");
    static constexpr int RPP = RPW < CHUNKS / 64 ? RPW : CHUNKS / 64;  // a wave's runs per page
    static constexpr int NPW = RPW / RPP;                               // pages a wave loads per step
    static_assert(RPW % RPP == 0, "a wave's runs cover whole pages or lie in one page");
};

// Chunk swizzle of a V row: rows 4g .. 4g + 3 (one transposed read) and the neighbouring four rows put the two
// chunks a 16-dim tile needs on distinct banks.  Even values only, so the two chunks of a tile stay adjacent.
template <int D>
__device__ __forceinline__ int v_swizzle(int t)
{
    return D == 64 ? 2 * ((t >> 1) & 3) : 2 * (t & 7);
}

// K swizzle: 16-byte chunk c of key row t sits at chunk c ^ k_swizzle<D>(t).  A K operand read takes the same
// chunk of 16 key rows, and 16 lanes of a 16-byte read are served per LDS cycle (256 bytes), so the 16 rows must
// land on distinct 16-byte slots of a 256-byte window: at head_dim 128 and 256 a row is a multiple of 256 bytes
// and the swizzle permutes all 16 chunk slots (with the 8 slots of the earlier 3-bit swizzle, every such read
// cost a 2-way conflict: LDS bank-conflict cycles equal to the product count); 128-byte rows (head_dim 64)
// alternate the window's halves by themselves.
template <int D>
__device__ __forceinline__ int k_swizzle(int t)
{
    if constexpr (D == 64)
        return (t & 7) ^ ((t >> 3) << 1);
    else
        return t & 15;
}

// 8-bit K rows (D bytes): the 16 rows of one 8-byte operand read (same chunk) on distinct banks.
template <int D>
__device__ __forceinline__ int k8_swizzle(int t)
{
    return D == 64 ? (t >> 2) & 3 : (D == 128 ? (t >> 1) & 7 : t & 15);
}

// 8-bit V rows: one transposed read takes chunk n of rows 4g .. 4g + 3 of two pages u0, u0 + 1 (u = page within
// the step); their chunk positions sit on distinct banks.
template <int D>
__device__ __forceinline__ int v8_swizzle(int t, int u)
{
    return D == 64 ? (u & 1) : (D == 128 ? (((t >> 1) & 3) | ((u & 1) << 2)) : ((t & 3) | ((u & 1) << 2)));
}

// One 16-byte global -> LDS load per lane: lane l's 16 bytes from `src` land at LDS address `dst` + 16 * l (dst
// uniform).  Issued as inline assembly so the compiler does not track it: its own waits would otherwise hold
// every LDS read behind every load in flight, whichever stage it writes.  The kernel waits for these loads
// itself (wait_vm) before the barrier that publishes a stage, and M0 is used by nothing else in the kernel.
__device__ __forceinline__ void load_lds16(const void* src, const FFKV_LDS void* dst)
{
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)))
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// The same load with a uniform 64-bit base and a 32-bit per-lane byte offset (no per-lane address arithmetic).
__device__ __forceinline__ void load_lds16(const void* base, uint32_t offset, const FFKV_LDS void* dst)
{
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    const uint64_t b64 = reinterpret_cast<uint64_t>(base);
    // readfirstlane returns int: go through uint32_t so the low word is not sign-extended into the high word
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b64)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b64 >> 32)));
    const uint64_t sb = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(offset), "s"(sb), "s"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)))
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// One 4-byte global -> LDS load per lane (lane l's word lands at `dst` + 4 * l).
__device__ __forceinline__ void load_lds4(const void* src, const FFKV_LDS void* dst)
{
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(src), "s"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)))
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// 8-bit caches: a wave issuing matrix products (with the operand conversions between them) runs at raised
// priority, so the SIMD's other wave fills the issue slots around them with its softmax instead of competing for
// the products' turn (measured: C4-shaped fp8 prefill 361 -> 314 us, int8 441 -> 403 us; 16-bit caches, whose
// operands need no conversion, are 1-3 % slower with it and leave it off).
template <bool ON>
__device__ __forceinline__ void mfma_priority(int level)
{
    if constexpr (ON)
    {
        if (level) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    }
}

// Wait for this wave's LDS operations (and scalar loads), leaving the vector-memory counter alone.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14)); }

template <int VM>
__device__ __forceinline__ void wait_vm()
{
    static_assert(VM >= 0 && VM < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(VM | (0x7 << 4) | (0xF << 8));  // vmcnt(VM), expcnt and lgkmcnt not waited on
}

}  // namespace

// PFX = false: prefill (the contract above).  PFX = true: split-K partials of decode queries over a prefix of
// pages shared by every row (pages 0 .. pfx_blocks - 1 of row 0's block table, which all rows hold): one query
// per (row, head), attending keys 0 .. min(ctx + 1, prefix) - 1, written as (max, denominator, unnormalised
// output) to the decode workspace for the decode merge to fold in.
// RG: row groups per wave.  A wave holds RG x 16 query rows; every K and V^T operand it reads from LDS feeds RG
// matrix products, so RG = 2 halves the LDS reads and the per-step scalar work per query row (4 waves of 32 rows
// instead of 8 waves of 16, two waves per SIMD).
// Register budget: 256 at two row groups (two waves per SIMD); one row group at head_dim <= 128 takes 128 (four waves
// per SIMD), or 168 for int8 codes, whose scales and conversions would spill at 128.
// LDS of one workgroup: kDmaStages<D> stages, each [K tile | V tile | int8 scales] of KP pages, key-major, swizzled
// chunks (stages past kDmaStages<D> take 16 bytes).
template <int QT, int D, int CT, bool PFX, int RG>
struct PrefillLds
{
    static constexpr bool C16 = FFKV_PREFILL_C16 && CT == I8 && !(FFKV_PREFILL_I8_BF && QT != F16) && D <= 128;
    using C = DmaCfg<D, C16 ? 2 : kElemBytes<CT>, CT == I8, 8 / RG, PFX>;
    static constexpr int STAGE = 2 * C::TILEB + C::SCB;
    static constexpr int S2 = kDmaStages<D> >= 3 ? STAGE : 16;
    static constexpr int S3 = kDmaStages<D> == 4 ? STAGE : 16;
    static constexpr int BYTES = 2 * STAGE + S2 + S3;  // the four in a row
    static_assert(BYTES + 16 <= 160 * 1024,
                  "the stages exceed the 160 KiB of LDS of a CU: fewer stages (FFKV_PREFILL_STAGES) or pages per step "
                  "(FFKV_PREFILL_DMA_KP*) for this head_dim");
};

// One workgroup's share of a prefill (or of the shared-prefix partials): `wg_index` is its index in the launch grid
// (blockIdx.x for paged_prefill_dma), s_st0 .. s_st3 its LDS stages (16-byte aligned, PrefillLds<...>::STAGE, S2 and
// S3 bytes) and `s_vover` an int in LDS.  Every wave of the workgroup calls it; it leaves no load in flight into
// the stages.  (paged_prefill_dma gives each stage an LDS array of its own, which tells the compiler that they
// do not overlap.)
template <int QT, int D, int CT, bool PFX, int RG>
__device__ __forceinline__ void prefill_wg(PrefillArgs a, int wg_index, uint8_t* s_st0, uint8_t* s_st1,
                                           uint8_t* s_st2, uint8_t* s_st3, int& s_vover)
{
    constexpr int  W = 8 / RG;  // waves per workgroup
    constexpr int  EB = kElemBytes<CT>;
    constexpr bool Q8 = EB == 1;
    // int8 codes are exact in bf16 and f16 alike; beside a bf16 q they take f16 products (QX16 below) unless
    // FFKV_PREFILL_I8_BF selects bf16 ones (q whole, codes converted through fp32)
    constexpr bool BF = CT == I8 ? (FFKV_PREFILL_I8_BF && QT != F16) : kBF<CT, QT>;
    // int8 with a bf16 q and f16 score products (QX16): q converts to f16 exactly (8 significant bits fit in 11),
    // scaled by a power of two when the wave's largest |q| would not fit f16's range, so it needs no lo part, and
    // the codes convert to f16 with the one-instruction bias trick instead of through fp32.
    constexpr bool QX16 = CT == I8 && QT == BF16 && !BF;
    // int8 pages with f16 score products at head_dim <= 128 (C16): the loads land the codes in LDS and each wave
    // converts the runs it loaded to f16, into the 16-bit tile layout, before the step's barrier; the products then
    // read f16 tiles as for an f16 cache, where otherwise every wave converts every K and V operand it reads (the
    // whole tile).  The 16-bit tiles take twice the LDS, which head_dim 256 cannot spare.
    constexpr bool C16 = FFKV_PREFILL_C16 && CT == I8 && !BF && D <= 128;
    constexpr bool R8 = Q8 && !C16;  // tiles read from LDS as 8-bit codes
    // LC: the load runs over the pages' bytes; C: the LDS tiles (16-bit for C16).  The scale bytes (and their
    // loads, counted in the waits) only for int8.
    using LC = DmaCfg<D, EB, CT == I8, W, PFX>;
    using C = DmaCfg<D, C16 ? 2 : EB, CT == I8, W, PFX>;
    using M = MType<BF>;
    using X8 = typename M::x8;
    constexpr int  KP = C::KP;
    constexpr int  KSTEPS = D / 32;
    constexpr int  NT = D / 16;
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF) || QX16);
    // Load issue per page (one table select and page base per page, then the page's runs) or per run (a 64-bit
    // page-offset select per run).  The per-page form has a third less scalar work and measured 1-6 % faster on the
    // chunked prefill for every cache type and head_dim (since the f16 PV products of 8-bit caches, bf16 queries
    // over bf16 / fp8 caches at head_dim 128 too, where the per-run form had been 2-3 % ahead); the shared-prefix
    // partials keep the per-run form.
    constexpr bool PAGE_ISSUE = !PFX;
    // 8-bit codes are exact in f16 as in bf16: with bf16 score products (BF), their PV products still take f16
    // V^T and P^T, so P needs one product instead of a bf16 hi + lo pair.
    constexpr bool V16 = FFKV_PREFILL_V16 && Q8 && BF;
    // f16 P (f16 caches, the f16 PV products of fp8 caches, and bf16 pages' f16 V tiles, VCONV below): the
    // denominator sums the rounded P that the products take, two values per v_dot2_f32_f16, in place of one add
    // per p.  int8's P carries the keys' V scales, so its denominator sums p itself, as do bf16's hi + lo pairs.
    constexpr bool L_DOT = !(BF && !V16) && CT != I8;
    // fp8 pages (operands converted as they are read): that denominator as one more product per 32 keys with a V^T
    // tile of ones, whose every output holds the column's sum, in place of the dot products (C4-shaped fp8
    // prefill 210.9 -> 206.7 us; bf16 and f16 pages gained nothing from it)
    constexpr bool L_MFMA = FFKV_PREFILL_L_MFMA && R8;

    static_assert(PrefillLds<QT, D, CT, PFX, RG>::STAGE == 2 * C::TILEB + C::SCB, "stage layout");
    // s_vover: some accumulator is not finite after the f16 PV products (bf16 and int8 pages)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid == 0) s_vover = 0;
    const int c = lane & 15;
    const int g = lane >> 4;
    // Workgroup -> (group, row block).  A group is (row b, kv head) for prefill and (kv head, chunk of prefix
    // pages) for prefix partials.  Consecutive workgroups go to the eight XCDs in turn; every row block of one
    // group is given to the same XCD, so the group's pages are fetched into one L2, not eight.  The longest work
    // goes out first, which shortens the tail (2-5 % on an 8 x 512-token chunk): an XCD's groups by decreasing
    // cached length, and a group's row blocks last first (the later prefill tokens see the most keys).
    const int G = a.group;
    const int S = a.seq_len;
    const int Hq = a.num_heads;
    const int Hkv = a.num_kv_heads;
    const int R = PFX ? a.batch * G : S * G;  // query rows of a group: (token, head) or (row, head) pairs
    const int nrb = (R + kDmaRows - 1) / kDmaRows;
    const int groups = PFX ? Hkv * a.pfx_chunks : a.batch * Hkv;
#if FFKV_PREFILL_XCD
    const int wg = wg_index;
    const int xcd = wg % kXcds;
    const int k_in_xcd = wg / kXcds;
    const int rb = nrb - 1 - k_in_xcd % nrb;
    int       grp = (k_in_xcd / nrb) * kXcds + xcd;
    const int g8 = (groups + kXcds - 1) / kXcds;  // group slots of this XCD: groups j * kXcds + xcd, j < g8
    if (!PFX && a.paged && g8 <= 64 && g8 > 1)
    {
        // The XCD's groups by decreasing cached length (ties by index): lane j ranks group j * kXcds + xcd, and
        // the workgroup takes the group ranked k_in_xcd / nrb.  Absent groups (past `groups`) rank last.
        const int gl = lane * kXcds + xcd;
        const int wl = lane < g8 && gl < groups ? a.context_lens[gl / a.num_kv_heads] : -2147483647 - 1;
        int       rank = 0;
        for (int m = 0; m < g8; ++m)
        {
            const int wm = __builtin_amdgcn_readlane(wl, m);
            rank += (wm > wl || (wm == wl && m < lane)) ? 1 : 0;
        }
        const uint64_t hit = __ballot(lane < g8 && rank == k_in_xcd / nrb);
        grp = hit != 0 ? (__ffsll(static_cast<long long>(hit)) - 1) * kXcds + xcd : groups;
    }
    if (grp >= groups) return;  // padding of the grid to whole rounds of XCDs
#else
    const int grp = wg_index / nrb;
    const int rb = wg_index % nrb;
#endif
    const int b = PFX ? 0 : grp / Hkv;                 // prefill: the workgroup's row
    const int kvh = PFX ? grp / a.pfx_chunks : grp % Hkv;
    const int chunk = PFX ? grp % a.pfx_chunks : 0;  // prefix: pages chunk*pfx_chunk_pages ..
    const int row0 = rb * kDmaRows;
    if (row0 >= R) return;  // uniform over the workgroup

    // This lane's query rows (MFMA columns), one per row group gi: row r = row0 + 16 (RG wave + gi) + c is
    // prefill token t of row b, head h, or for the prefix its decode query of row bq, head h.  It sees keys
    // [0, kend).  Pages pg_lo .. pg_hi - 1 are the workgroup's; rows 0 .. L - 1 of them hold keys (the rest load
    // as zeros).
    bool   col_ok[RG];
    int    hq[RG], kend[RG], bq[RG];
    size_t qrow[RG];
    int    L, pg_lo, pg_hi;
    int64_t ctx = 0;
    if constexpr (PFX)
    {
        L = a.pfx_blocks * kBlockSize;
        pg_lo = chunk * a.pfx_chunk_pages;
        pg_hi = min(pg_lo + a.pfx_chunk_pages, a.pfx_blocks);
    }
    else
    {
        ctx = a.paged ? static_cast<int64_t>(a.context_lens[b]) : 0;
        int64_t Lr = ctx + S;
        if (a.paged && Lr > a.cap_tokens) Lr = a.cap_tokens;
        if (Lr < 0) Lr = 0;
        L = __builtin_amdgcn_readfirstlane(static_cast<int>(Lr));
    }
#pragma unroll
    for (int gi = 0; gi < RG; ++gi)
    {
        const int r = row0 + 16 * (RG * wave + gi) + c;
        col_ok[gi] = r < R;
        hq[gi] = kvh * G + (col_ok[gi] ? r % G : 0);
        if constexpr (PFX)
        {
            bq[gi] = col_ok[gi] ? r / G : 0;
            int64_t ke = static_cast<int64_t>(a.context_lens[bq[gi]]) + 1;  // the decode query sees ctx + 1 keys
            if (ke > a.cap_tokens) ke = a.cap_tokens;
            ke = ke > L ? L : (ke < 0 ? 0 : ke);
            kend[gi] = col_ok[gi] ? static_cast<int>(ke) : 0;
            qrow[gi] = static_cast<size_t>(bq[gi]) * Hq + hq[gi];
        }
        else
        {
            bq[gi] = 0;
            const int t = col_ok[gi] ? r / G : 0;
            int64_t   ke = ctx + t + 1;
            ke = ke > L ? L : (ke < 0 ? 0 : ke);
            kend[gi] = col_ok[gi] ? static_cast<int>(ke) : 0;
            qrow[gi] = (static_cast<size_t>(b) * S + t) * Hq + hq[gi];
        }
    }
    if constexpr (!PFX)
    {
        const int r_last = min(row0 + kDmaRows, R) - 1;
        int64_t   kw = ctx + r_last / G + 1;
        kw = kw > L ? L : (kw < 0 ? 0 : kw);
        pg_lo = 0;
        pg_hi = static_cast<int>((kw + kBlockSize - 1) / kBlockSize);
    }
    // uniform values computed through divisions: keep them scalar so the loop's branches stay scalar
    pg_lo = __builtin_amdgcn_readfirstlane(pg_lo);
    pg_hi = __builtin_amdgcn_readfirstlane(pg_hi);
    const int  steps = pg_hi > pg_lo ? (pg_hi - pg_lo + KP - 1) / KP : 0;
    const bool wave_active = row0 + 16 * RG * wave < R;

    // ---- Q^T operands of the wave's RG x 16 query rows -----------------------------------------------------
    X8    qhi[RG][KSTEPS], qlo[RG][KSTEPS];
    float q_unscale = 1.0f;  // QX16: the scores come out scaled by 1 / q_unscale
    if constexpr (QX16)
    {
        float x[RG][KSTEPS][8];
        float amax = 0.0f;
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
            {
                if (col_ok[gi])
                    load_q8<QT>(a.q, qrow[gi] * D + 32 * j + 8 * g, x[gi][j]);
                else
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[gi][j][e] = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) amax = fmaxf(amax, __builtin_fabsf(x[gi][j][e]));
            }
        amax = group_max<32>(fmaxf(amax, __shfl_xor(amax, 32, 64)));  // the wave's largest |q| (NaN skipped)
        float qs = 1.0f;
        if (__builtin_expect(amax >= 32768.0f, 0))  // uniform: scale q into f16's range by a power of two
        {
            const int e = __builtin_amdgcn_frexp_expf(amax);  // amax < 2^e
            qs = __builtin_ldexpf(1.0f, 15 - e);              // amax * qs < 2^15
            q_unscale = __builtin_ldexpf(1.0f, e - 15);
        }
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
            {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                            f32x2{x[gi][j][2 * e] * qs, x[gi][j][2 * e + 1] * qs}, h2));
                qhi[gi][j] = qlo[gi][j] = __builtin_bit_cast(X8, u32x4{w[0], w[1], w[2], w[3]});
            }
    }
    else
#pragma unroll
    for (int gi = 0; gi < RG; ++gi)
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            const int d0 = 32 * j + 8 * g;
            if constexpr (!NEED_LO)
            {
                u32x4 w = u32x4{0u, 0u, 0u, 0u};
                if (col_ok[gi])
                    w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + qrow[gi] * D + d0);
                qhi[gi][j] = __builtin_bit_cast(X8, w);
                qlo[gi][j] = qhi[gi][j];
            }
            else
            {
                float x[8];
                if (col_ok[gi])
                    load_q8<QT>(a.q, qrow[gi] * D + d0, x);
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
                qhi[gi][j] = __builtin_bit_cast(X8, u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                                          hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)});
                qlo[gi][j] = __builtin_bit_cast(X8, u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                                          lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)});
            }
        }

    if constexpr (CT == FP8)
    {
        // A negative K scale negates every score: q's signs are flipped once here instead of the scores at every
        // step (exact: a sign flip commutes with the products and their rounding).
        if (a.k_scale[kvh] < 0.0f)
#pragma unroll
            for (int gi = 0; gi < RG; ++gi)
#pragma unroll
                for (int j = 0; j < KSTEPS; ++j)
                {
                    qhi[gi][j] = __builtin_bit_cast(X8, __builtin_bit_cast(u32x4, qhi[gi][j]) ^ 0x80008000u);
                    qlo[gi][j] = __builtin_bit_cast(X8, __builtin_bit_cast(u32x4, qlo[gi][j]) ^ 0x80008000u);
                }
    }

    // Nothing else is in flight from here on but the page loads: the pipeline's waits count only those.
    wait_vm<0>();

    // ---- loads: wave w fetches runs w*RPW .. w*RPW + RPW - 1 (64 chunks each) of the K tile and of the V tile --
    // (bf16 pages, whose V tiles are converted to f16 in LDS (VCONV): wave w fetches runs w*RPW/2 ..
    // w*RPW/2 + RPW/2 - 1 of the K tile and the same runs of the V tile, so that every wave converts the same share)
    constexpr bool VCONV = FFKV_PREFILL_VCONV && CT == BF16;
    static_assert(!VCONV || LC::RPW % 2 == 0, "a wave loads as many V runs as K runs");
    constexpr int RPP = VCONV ? (LC::RPW / 2 < LC::CHUNKS / 64 ? LC::RPW / 2 : LC::CHUNKS / 64) : LC::RPP;  // runs per page
    constexpr int NPW = LC::RPW / RPP;  // pages (or parts of one) a wave loads per step
    static_assert(LC::RPW % RPP == 0 && (!VCONV || (LC::RPW / 2) % RPP == 0), "a wave's runs cover whole page parts");
    auto run_is_v = [&](int k) { return VCONV ? k >= LC::RPW / 2 : wave * LC::RPW + k >= LC::IPR; };
    auto run_lr = [&](int k)
    {
        if constexpr (VCONV) return wave * (LC::RPW / 2) + (k >= LC::RPW / 2 ? k - LC::RPW / 2 : k);
        const int run = wave * LC::RPW + k;
        return run >= LC::IPR ? run - LC::IPR : run;
    };
    const FFKV_CONST int32_t* table_row =  // prefix: row 0's table, whose first pfx_blocks entries every row shares
        a.paged ? (const FFKV_CONST int32_t*)(a.block_table + static_cast<int64_t>(b) * a.max_blocks) : nullptr;
    const char* zero_src = reinterpret_cast<const char*>(g_zero_chunks) + 16 * lane;
    // Wave w loads runs w*RPW .. w*RPW + RPW - 1 of the step (runs 0 .. IPR - 1 are K, the rest V).  Per-lane part
    // of each load's source, the same for every page: key row `tok` of the page, chunk `ch` (swizzled to where
    // this lane's 16 bytes land), as a byte offset from the page's (row, kv head) base.
    uint32_t voff[LC::RPW];
    int      vtok[LC::RPW];
#pragma unroll
    for (int k = 0; k < LC::RPW; ++k)
    {
        const bool is_v = run_is_v(k);                     // uniform
        const int  lr = run_lr(k);                          // run within its tile
        const int  u = lr * 64 / LC::CHUNKS;                 // page of the step
        const int  p = lr * 64 % LC::CHUNKS + lane;          // chunk position within the page
        const int  tok = p / LC::CPT;
        int        sw;
        if constexpr (C16)
            sw = 0;  // landed in order: the conversion puts the chunks in place
        else if constexpr (Q8)
            sw = is_v ? v8_swizzle<D>(tok, u) : k8_swizzle<D>(tok);
        else
            sw = is_v ? v_swizzle<D>(tok) : k_swizzle<D>(tok);
        const int ch = (p % LC::CPT) ^ sw;
        vtok[k] = tok;
        voff[k] = static_cast<uint32_t>(tok * Hkv * LC::RB + 16 * ch);
    }
    const size_t row_bytes = static_cast<size_t>(Hkv) * LC::RB;  // one key row of all kv heads

    // A wave's runs j*RPP .. j*RPP + RPP - 1 lie in one page of one tile (per-page issue).
    // Per-run constants of this wave's loads (uniform): source tensor at kv head kvh, page of the step, LDS
    // destination.  A page's byte offset is row_base + index * page_bytes, with index the physical page (paged) or
    // the page of the row (contiguous keys).
    const char* run_src[LC::RPW];
    int         run_u[LC::RPW];
    int         run_dst[LC::RPW];
#pragma unroll
    for (int k = 0; k < LC::RPW; ++k)
    {
        const bool is_v = run_is_v(k);
        const int  lr = run_lr(k);
        run_u[k] = lr * 64 / LC::CHUNKS;
        run_src[k] = static_cast<const char*>(is_v ? a.v_cache : a.k_cache) + static_cast<size_t>(kvh) * LC::RB;
        // C16: run lr's codes land in the upper half of the 2 KiB its rows take in the 16-bit tile
        run_dst[k] = (is_v ? C::TILEB : 0) + (C16 ? lr * 2048 + 1024 : lr * 64 * 16);
    }
    // C16: where this lane's 16 codes go once converted (the 16-bit chunks 2ch and 2ch + 1 of its key row, at
    // their swizzled places), relative to run_dst[k].  A scattered 16-byte LDS write is served 8 lanes at a time
    // over 128 bytes, so the 8 lanes of each group must write 8 distinct 16-byte slots modulo 128 bytes: with the
    // lower half of every lane's codes written first, a group (4 chunks of one or two key rows) fills the slots
    // of one parity only (two lanes per bank group: 8 conflict cycles per write, one per matrix product).  Lanes
    // 4..7 of each group therefore write the other parity first: c16_hi1[k] says the lane's first write holds
    // its upper 8 values.
    int  c16_dst[C16 ? LC::RPW : 1][2];
    bool c16_hi1[C16 ? LC::RPW : 1];
    if constexpr (C16)
#pragma unroll
        for (int k = 0; k < LC::RPW; ++k)
        {
            const int p = run_lr(k) * 64 % LC::CHUNKS + lane;
            const int tok = p / LC::CPT;
            const int ch = p % LC::CPT;
            const int sw = run_is_v(k) ? v_swizzle<D>(tok) : k_swizzle<D>(tok);
            const int hs = ((lane >> 2) ^ sw) & 1;  // the first write's slot has parity (lane >> 2) & 1
            c16_hi1[k] = hs != 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) c16_dst[k][h] = 32 * (lane - ch) - 1024 + 16 * ((2 * ch + (h ^ hs)) ^ sw);
        }
    const uint32_t page_bytes = static_cast<uint32_t>(kBlockSize * row_bytes);
    const uint64_t row_base = a.paged ? 0 : static_cast<uint64_t>(b) * S * row_bytes;

    // Requests step si into `stage`; returns its page mask (bit u: page pg_lo + si*KP + u is present; keys on absent
    // pages are masked).  Block-table entries are uniform and come through the scalar cache.  Pages whose 16
    // rows are all keys of the row load with a uniform base; the row's last, partial page (and absent pages)
    // fetch the zero block for the missing rows.  The scalar work is kept short: it runs once per step in every
    // wave, in order with the wave's matrix and vector work.
    auto issue = [&](int si, uint8_t* stage) -> int
    {
        int      okm = 0, full = 0;
        uint64_t page_off[KP];
        uint32_t page_row[KP];  // physical page of present pages (int8 scales are indexed by it), else 0
#pragma unroll
        for (int u = 0; u < KP; ++u)
        {
            const int pg = pg_lo + si * KP + u;
            uint32_t  idx = 0;
            bool      present = false;
            if (pg < pg_hi)  // pg_hi <= max_blocks
            {
                if (a.paged)
                {
                    idx = static_cast<uint32_t>(table_row[pg]);
                    present = idx < static_cast<uint32_t>(a.num_blocks);  // negative entries are absent
                }
                else
                {
                    idx = static_cast<uint32_t>(pg);
                    present = true;
                }
            }
            idx = present ? idx : 0u;
            page_row[u] = idx;
            page_off[u] = row_base + static_cast<uint64_t>(idx) * page_bytes;
            okm |= present ? 1 << u : 0;
            full |= present && (pg + 1) * kBlockSize <= L ? 1 << u : 0;
        }
        if constexpr (PAGE_ISSUE)
        {
#pragma unroll
            for (int j = 0; j < NPW; ++j)
            {
                const int u = run_u[j * RPP];
                uint32_t  idx = page_row[0];  // page_row[u] without a dynamic index (u is uniform, not constant)
#pragma unroll
                for (int uu = 1; uu < KP; ++uu) idx = u == uu ? page_row[uu] : idx;
                const char* base = run_src[j * RPP] + row_base + static_cast<uint64_t>(idx) * page_bytes;
                const bool  fl = (full >> u) & 1;
                const bool  pres = (okm >> u) & 1;
                const int   tok0 = (pg_lo + si * KP + u) * kBlockSize;
                if (fl)
                {
#pragma unroll
                    for (int r = 0; r < RPP; ++r)
                    {
                        const int k = j * RPP + r;
                        load_lds16(base, voff[k], (const FFKV_LDS void*)(stage + run_dst[k]));
                    }
                }
                else
                {
#pragma unroll
                    for (int r = 0; r < RPP; ++r)
                    {
                        const int  k = j * RPP + r;
                        const bool take = pres && tok0 + vtok[k] < L;
                        load_lds16(take ? static_cast<const void*>(base + voff[k]) : static_cast<const void*>(zero_src),
                                   (const FFKV_LDS void*)(stage + run_dst[k]));
                    }
                }
            }
        }
        else
        {
#pragma unroll
            for (int k = 0; k < LC::RPW; ++k)
            {
                const int u = run_u[k];
                uint64_t  poff = page_off[0];  // page_off[u] without a dynamic index (u is uniform but not constant)
#pragma unroll
                for (int uu = 1; uu < KP; ++uu) poff = u == uu ? page_off[uu] : poff;
                const char*          base = run_src[k] + poff;
                const FFKV_LDS void* dst = (const FFKV_LDS void*)(stage + run_dst[k]);
                if ((full >> u) & 1)
                {
                    load_lds16(base, voff[k], dst);
                }
                else
                {
                    const bool take = ((okm >> u) & 1) && (pg_lo + si * KP + u) * kBlockSize + vtok[k] < L;
                    load_lds16(take ? static_cast<const void*>(base + voff[k]) : static_cast<const void*>(zero_src), dst);
                }
            }
        }
        if constexpr (CT == I8)
        {
            // the step's per-token scales, K then V: lane l of run s takes scale l + 64 s (every wave issues the same
            // loads, so every wave's wait counts match; the copies write the same values)
#pragma unroll
            for (int sr = 0; sr < C::SCB / 256; ++sr)
            {
                const int  e = lane + 64 * sr;
                const bool is_v = e >= KP * kBlockSize;
                const int  u = (e / kBlockSize) % KP;
                const int  t = e % kBlockSize;
                uint32_t   pr = page_row[0];
#pragma unroll
                for (int uu = 1; uu < KP; ++uu) pr = u == uu ? page_row[uu] : pr;
                const bool take = ((okm >> u) & 1) && (pg_lo + si * KP + u) * kBlockSize + t < L;
                const float* src = (is_v ? a.v_scale : a.k_scale) +
                                   (static_cast<size_t>(pr) * kBlockSize + t) * Hkv + kvh;
                load_lds4(take ? static_cast<const void*>(src) : static_cast<const void*>(zero_src),
                          (const FFKV_LDS void*)(stage + 2 * C::TILEB + 256 * sr));
            }
        }
        return okm;
    };

    // ---- compute ---------------------------------------------------------------------------------------------
    // Online softmax on raw scores: m_run is the column's reference maximum (raw units), p = 2^(s*c - m_run*c)
    // with c = scale * log2(e).  The reference moves (and acc / l_run are rescaled) only when a new maximum
    // exceeds it by more than 8 / c, so p stays below 2^8 and most steps rescale nothing; numerator and
    // denominator share the reference, so the result is the same softmax.
    float c_log2 = a.scale_log2 * q_unscale;
    float v_head_scale = 1.0f;
    if constexpr (CT == FP8)  // per-head scales: K's into the score scale (its sign into q), V's onto the output
    {
        const float ks = a.k_scale[kvh];
        // a zero scale (every score 0: uniform weights, as in decode) keeps a tiny positive factor, so the raw
        // reference maximum, its threshold and masked keys' -inf scores stay well defined
        c_log2 = fmaxf(c_log2 * __builtin_fabsf(ks), 1e-30f);
        v_head_scale = a.v_scale[kvh];
    }
    const float thr_raw = 8.0f / c_log2;
    // int8 pages: on the rerun below every p is scaled by 2^kRerunShift, numerator and denominator alike, so the
    // result is the same softmax
    constexpr float kRerunShift = -12.0f;
    float       m_run[RG], l_run[RG];
    f32x4       lacc[RG];  // L_MFMA: the denominator's product (every element holds the column's sum)
    float       m_thr[RG], m_neg[RG];  // m_run + thr_raw, and -m_run * c_log2 (0 before the first key)
    f32x4       acc[RG][NT];

    // Smallest causal limit over the wave's active columns: steps wholly below it need no mask.
    int kmin = INT32_MAX;
#pragma unroll
    for (int gi = 0; gi < RG; ++gi) kmin = col_ok[gi] ? min(kmin, kend[gi]) : kmin;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) kmin = min(kmin, __shfl_xor(kmin, off, 64));
    kmin = __builtin_amdgcn_readfirstlane(kmin);

    // 16-bit K operand of k-step j: key c, dims 32j + 8g .. +8, chunk (4 j + g) ^ ksw of the key's row, at bytes
    // kb4[j % 4] + 64 (j - j % 4) (the swizzle's upper bits XOR j % 4)
    const int ksw = k_swizzle<D>(c);
    int       kb4[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) kb4[m] = 2 * (c * D + 8 * (g ^ (ksw & 3)) + 32 * (m ^ (ksw >> 2)));
    // 16-bit V^T operand via transposed reads: this lane supplies dims 16n + 4q .. +3 of key row 4g + rr of a page
    const int vrow = 4 * g + (c >> 2);
    const int vsw = v_swizzle<D>(vrow) >> 1;
    const int vbase = C::TILEB + 2 * (vrow * D + 4 * (c & 3));  // bytes
    // 8-bit K operand: 8 codes of key c at dims 32j + 8g: chunk 2j + g/2 (swizzled), half g & 1
    const int k8sw = k8_swizzle<D>(c);
    const int k8base = c * C::RB + 8 * (g & 1);
    // 8-bit V^T operand: lanes 2r, 2r + 1 supply the halves of chunk n of row r; rows 0..3 are keys 4g .. 4g + 3 of
    // page u0, rows 4..7 the same keys of page u0 + 1 (k-slots 8g + r)
    const int v8key = 4 * g + ((c >> 1) & 3);
    const int v8pg = (c >> 1) >> 2;  // 0: page u0, 1: page u0 + 1
    const int v8sw = v8_swizzle<D>(v8key, v8pg);
    const int v8base = C::TILEB + v8pg * kBlockSize * C::RB + v8key * C::RB + 8 * (c & 1);

    // S^T tiles of a step: scores of the wave's RG x 16 columns against the step's KP pages
    auto qk = [&](const uint8_t* stage, f32x4 (&s)[RG][KP])
    {
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
#pragma unroll
            for (int u = 0; u < KP; ++u) s[gi][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        auto kread = [&](int j, int u) -> X8
        {
            if constexpr (R8)
            {
                const int   ka = u * kBlockSize * C::RB + k8base + (((2 * j + (g >> 1)) ^ k8sw) << 4);
                // volatile: the compiler would pair the reads of pages u and u + 1 (2 KiB apart) into one
                // ds_read2st64_b64, whose two halves land on the same banks (one LDS conflict cycle per product,
                // measured; separate reads count none)
                const u32x2 w = *(const volatile FFKV_LDS u32x2*)(stage + ka);
                return __builtin_bit_cast(X8, codes_to_m<CT, BF>(w[0], w[1]));
            }
            else
            {
                const int ka = kb4[j & 3] + 64 * (j & ~3);
                return __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(stage + u * kBlockSize * C::RB + ka));
            }
        };
        // every K operand read from LDS feeds the products of all RG row groups
        mfma_priority<R8>(1);
        X8 kc[KP];
#pragma unroll
        for (int u = 0; u < KP; ++u) kc[u] = kread(0, u);
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            X8 kn[KP];
#pragma unroll
            for (int u = 0; u < KP; ++u) kn[u] = j + 1 < KSTEPS ? kread(j + 1, u) : kc[u];  // next k-step in flight
#pragma unroll
            for (int u = 0; u < KP; ++u)
#pragma unroll
                for (int gi = 0; gi < RG; ++gi)
                {
                    s[gi][u] = M::mma32(kc[u], qhi[gi][j], s[gi][u]);
                    if constexpr (NEED_LO) s[gi][u] = M::mma32(kc[u], qlo[gi][j], s[gi][u]);
                }
#pragma unroll
            for (int u = 0; u < KP; ++u) kc[u] = kn[u];
        }
        mfma_priority<R8>(0);
        if constexpr (CT == I8)  // per-token K scales of keys 4g .. 4g + 3 of each page
        {
#pragma unroll
            for (int u = 0; u < KP; ++u)
            {
                const f32x4 ksc = *reinterpret_cast<const f32x4*>(stage + 2 * C::TILEB + (u * kBlockSize + 4 * g) * 4);
#pragma unroll
                for (int gi = 0; gi < RG; ++gi) s[gi][u] *= ksc;
            }
        }
    };

    // Online softmax of a step's scores: the probabilities pv (int8: times the keys' V scales).
    auto softmax = [&]<bool VC, bool SH>(int si, const uint8_t* stage, int okm, f32x4 (&s)[RG][KP],
                                         float (&pv)[RG][KP * 4])
    {
        constexpr bool LD = L_DOT || VC;  // the f16 P of converted bf16 V tiles sums by dot products too
        const int pg0 = pg_lo + si * KP;
        // uniform: every key of the step is visible to every column of the wave
        const bool unmasked = okm == (1 << KP) - 1 && (pg0 + KP) * kBlockSize <= kmin;
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
        {
            // the scores are masked in place, so both paths leave them in the product registers (no copies)
            if (!unmasked)
            {
                const int kr = kend[gi] - pg0 * kBlockSize - 4 * g;  // key 4g + i of page u visible iff 16u + i < kr
#pragma unroll
                for (int u = 0; u < KP; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        const bool vis = ((okm >> u) & 1) && u * kBlockSize + i < kr;
                        s[gi][u][i] = vis ? s[gi][u][i] : kNegInf;
                    }
            }
            float sc[KP * 4];
            float mt = kNegInf;
#pragma unroll
            for (int u = 0; u < KP; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    sc[4 * u + i] = s[gi][u][i];
                    mt = fmaxf(mt, sc[4 * u + i]);
                }
            // the lane's maximum decides whether any column needs a new reference; only then do the column
            // maxima cross the lanes (a column's 16 keys sit in 4 lanes)
            if (__any(mt > m_thr[gi]))  // false while the column has seen no key (mt = -inf)
            {
                mt = swap_max(mt);
                const bool  upd = mt > m_thr[gi];
                const float alpha = upd ? __builtin_amdgcn_exp2f((m_run[gi] - mt) * c_log2) : 1.0f;  // 0 at first
                l_run[gi] *= alpha;
                if constexpr (L_MFMA && LD) lacc[gi] *= alpha;
#pragma unroll
                for (int n = 0; n < NT; ++n) acc[gi][n] *= alpha;
                m_run[gi] = upd ? mt : m_run[gi];
                m_thr[gi] = m_run[gi] + thr_raw;
                m_neg[gi] = m_run[gi] == kNegInf ? 0.0f : -m_run[gi] * c_log2;  // no key yet: every p is 0
                if constexpr (SH) m_neg[gi] += kRerunShift;
            }
#pragma unroll
            for (int e = 0; e < KP * 4; ++e)
            {
                pv[gi][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], c_log2, m_neg[gi]));
                if constexpr (!LD) l_run[gi] += pv[gi][e];
            }
        }
        if constexpr (CT == I8)  // per-token V scales multiply P (the denominator keeps the unscaled p)
        {
#pragma unroll
            for (int u = 0; u < KP; ++u)
            {
                const f32x4 vsc = *reinterpret_cast<const f32x4*>(
                    stage + 2 * C::TILEB + ((KP + u) * kBlockSize + 4 * g) * 4);
#pragma unroll
                for (int gi = 0; gi < RG; ++gi)
#pragma unroll
                    for (int i = 0; i < 4; ++i) pv[gi][4 * u + i] *= vsc[i];
            }
        }
    };

    // O^T += V^T P^T from the stage.  V16: the products take f16 V^T (codes converted to f16) and P^T, with P in
    // one product (11 bits); otherwise bf16 P is a hi + lo pair, which keeps 16 significant bits in two products.
    auto pv_mma = [&]<bool V16>(const uint8_t* stage, const float (&pv)[RG][KP * 4])
    {
        constexpr bool PBF = BF && !V16;           // P^T and V^T operand type
        constexpr bool LD = L_DOT || (CT == BF16 && V16);  // bf16 pages with V tiles converted to f16
        using MP = MType<PBF>;
        using XP = typename MP::x8;
        auto vread = [&](int n, int u0) -> XP  // V^T operand of output tile n over pages u0, u0 + 1
        {
            if constexpr (R8)
            {
                const auto raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (FFKV_LDS i32x2*)(stage + u0 * kBlockSize * C::RB + v8base + ((n ^ v8sw) << 4)));
                const u32x2 w = __builtin_bit_cast(u32x2, raw);
                return __builtin_bit_cast(XP, codes_to_m<CT, PBF>(w[0], w[1]));
            }
            else
            {
                const int  off = vbase + 32 * (n ^ vsw);
                const auto a0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                    (FFKV_LDS bf16x4*)(stage + u0 * kBlockSize * C::RB + off));
                const auto a1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                    (FFKV_LDS bf16x4*)(stage + (u0 + 1) * kBlockSize * C::RB + off));
                const u32x2 w0 = __builtin_bit_cast(u32x2, a0);
                const u32x2 w1 = __builtin_bit_cast(u32x2, a1);
                return __builtin_bit_cast(XP, u32x4{w0[0], w0[1], w1[0], w1[1]});
            }
        };
#pragma unroll
        for (int u0 = 0; u0 < KP; u0 += 2)
        {
            // P^T operands: pairs of p rounded to the MFMA type (packed conversions); for bf16 also the residual
            // p - hi.
            XP phi[RG], plo[RG];
#pragma unroll
            for (int gi = 0; gi < RG; ++gi)
            {
                uint32_t ph[4], pl[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    const f32x2 v = f32x2{pv[gi][4 * u0 + 2 * e], pv[gi][4 * u0 + 2 * e + 1]};
                    if constexpr (PBF)
                    {
                        ph[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
                        const f32x2 r = f32x2{v[0] - __builtin_bit_cast(float, ph[e] << 16),
                                              v[1] - __builtin_bit_cast(float, ph[e] & 0xffff0000u)};
                        pl[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
                    }
                    else
                    {
                        const h2 hp = __builtin_convertvector(v, h2);
                        ph[e] = __builtin_bit_cast(uint32_t, hp);
                        pl[e] = 0u;
                        if constexpr (LD && !L_MFMA)
                            l_run[gi] = __builtin_amdgcn_fdot2(hp, h2{1, 1}, l_run[gi], false);
                    }
                }
                phi[gi] = __builtin_bit_cast(XP, u32x4{ph[0], ph[1], ph[2], ph[3]});
                plo[gi] = __builtin_bit_cast(XP, u32x4{pl[0], pl[1], pl[2], pl[3]});
            }
            // every V^T operand read from LDS feeds the products of all RG row groups
            mfma_priority<R8>(1);
            XP vcur = vread(0, u0);
#pragma unroll
            for (int n = 0; n < NT; ++n)
            {
                XP vnxt{};
                if (n + 1 < NT) vnxt = vread(n + 1, u0);  // next tile's reads in flight behind this tile's products
#pragma unroll
                for (int gi = 0; gi < RG; ++gi)
                {
                    acc[gi][n] = MP::mma32(vcur, phi[gi], acc[gi][n]);
                    if constexpr (PBF) acc[gi][n] = MP::mma32(vcur, plo[gi], acc[gi][n]);
                }
                vcur = vnxt;
                if constexpr (LD && L_MFMA)
                    if (n == 0)
                    {
                        const XP ones = __builtin_bit_cast(XP, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
#pragma unroll
                        for (int gi = 0; gi < RG; ++gi) lacc[gi] = MP::mma32(ones, phi[gi], lacc[gi]);
                    }
            }
            mfma_priority<R8>(0);
        }
    };

    // ---- pipeline: stage si % NS ---------------------------------------------------------------------------
    // Every step issues the same number of loads (steps past the end fetch the zero block into a stage nobody
    // reads), so "step si has landed" is always vmcnt <= the loads of steps si + 1 .. si + NS - 2.
    constexpr int NS = kDmaStages<D>;
    constexpr int LPS = LC::RPW + C::SCB / 256;  // loads per wave and step

    // bf16 pages (VCONV): every wave converts the V runs it loads to f16 in place, in LDS, as soon as its own loads
    // of them have landed and before the barrier that publishes the step; the PV products then take f16 V^T and P
    // in one product instead of bf16 P's hi + lo pair.  bf16 values are exact in f16 from 2^-14 to 65280 (below
    // 2^-14 they round to f16 subnormals, an absolute error of at most 2^-25).  A value of 65520 or more (or
    // infinite) becomes infinite and makes the accumulators infinite or NaN (p * inf, 0 * inf): the workgroup then
    // runs the whole pipeline again on the bf16 path.
    auto convert_v = [&](uint8_t* stage)
    {
#pragma unroll
        for (int k = LC::RPW / 2; k < LC::RPW; ++k)
        {
            auto* p = (FFKV_LDS u32x4*)(stage + run_dst[k] + 16 * lane);
            const u32x4 w = *p;
            u32x4       o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const float lo = __builtin_bit_cast(float, w[e] << 16);
                const float hi = __builtin_bit_cast(float, w[e] & 0xffff0000u);
                o[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, h2));
            }
            *p = o;
        }
    };

    // int8 pages (C16): every wave converts the runs it loads (K and V) to f16 in the 16-bit tile layout, as soon
    // as its own loads of them have landed and before the barrier that publishes the step.  A run's codes sit in
    // the upper half of the region its f16 values fill, which no other run touches; the whole run is read before
    // any of it is written.
    auto convert_c16 = [&](uint8_t* stage)
    {
#pragma unroll
        for (int k = 0; k < (C16 ? LC::RPW : 0); ++k)
        {
            const u32x4 w = *(FFKV_LDS u32x4*)(stage + run_dst[k] + 16 * lane);
            const bool  h1 = c16_hi1[k];
            const u32x4 first = codes_to_m<CT, false>(h1 ? w[2] : w[0], h1 ? w[3] : w[1]);
            const u32x4 second = codes_to_m<CT, false>(h1 ? w[0] : w[2], h1 ? w[1] : w[3]);
            *(FFKV_LDS u32x4*)(stage + run_dst[k] + c16_dst[k][0]) = first;
            *(FFKV_LDS u32x4*)(stage + run_dst[k] + c16_dst[k][1]) = second;
        }
    };

    // The scores' products are issued before the next loads' scalar address work, which then runs while they
    // execute.
    // With three or more stages, step si + 1 has been requested a step before step si is computed, so its tiles
    // are converted while step si's score products run (AH), instead of at the head of step si + 1.
    auto body = [&]<bool VC, bool SH>(int si, uint8_t* cur, int okm_cur, uint8_t* nxt, int& okm_nxt, uint8_t* ahead)
    {
        constexpr bool AH = FFKV_PREFILL_AHEAD && NS >= 3 && (VC || C16);
        wait_vm<(NS - 2) * LPS>();
        if constexpr (AH)
        {
            wait_lgkm0();  // this wave's conversion of step si (at step si - 1) is written before the barrier
        }
        else
        {
            if constexpr (VC)
            {
                convert_v(cur);
                wait_lgkm0();  // the converted runs are written before the barrier publishes them
            }
            if constexpr (C16)
            {
                convert_c16(cur);
                wait_lgkm0();
            }
        }
        __builtin_amdgcn_s_barrier();  // step si visible to all; every wave is past step si - 1 (stage of si+NS-1)
        f32x4 sx[RG][KP];
        if (wave_active) qk(cur, sx);
        if constexpr (AH)
        {
            wait_vm<(NS - 3) * LPS>();  // step si + 1 has landed (its stage's last readers were past step si - 1)
            if constexpr (VC) convert_v(ahead);
            if constexpr (C16) convert_c16(ahead);
        }
        okm_nxt = issue(si + NS - 1, nxt);
        if (wave_active)
        {
            float pv[RG][KP * 4];
            softmax.template operator()<VC, SH>(si, cur, okm_cur, sx, pv);
            pv_mma.template operator()<V16 || VC>(cur, pv);
        }
    };

    // VC: bf16 pages' V tiles converted to f16.  SH: int8 pages' p scaled by 2^kRerunShift (the rerun).
    auto pipeline = [&]<bool VC, bool SH>()
    {
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
        {
            m_run[gi] = kNegInf;
            m_thr[gi] = kNegInf;
            m_neg[gi] = 0.0f;
            l_run[gi] = 0.0f;
            lacc[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[gi][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        int okm0 = issue(0, s_st0);
        int okm1 = 0, okm2 = 0, okm3 = 0;
        if constexpr (NS >= 3) okm1 = issue(1, s_st1);
        if constexpr (NS == 4) okm2 = issue(2, s_st2);
        if constexpr (FFKV_PREFILL_AHEAD && NS >= 3 && (VC || C16))  // step 0's tiles, converted ahead of the loop
        {
            wait_vm<(NS - 2) * LPS>();
            if constexpr (VC) convert_v(s_st0);
            if constexpr (C16) convert_c16(s_st0);
        }
        for (int si = 0; si < steps; si += NS)
        {
            if constexpr (NS == 2)
            {
                body.template operator()<VC, SH>(si, s_st0, okm0, s_st1, okm1, s_st1);
                if (si + 1 >= steps) break;
                body.template operator()<VC, SH>(si + 1, s_st1, okm1, s_st0, okm0, s_st0);
            }
            else if constexpr (NS == 3)
            {
                body.template operator()<VC, SH>(si, s_st0, okm0, s_st2, okm2, s_st1);
                if (si + 1 >= steps) break;
                body.template operator()<VC, SH>(si + 1, s_st1, okm1, s_st0, okm0, s_st2);
                if (si + 2 >= steps) break;
                body.template operator()<VC, SH>(si + 2, s_st2, okm2, s_st1, okm1, s_st0);
            }
            else
            {
                body.template operator()<VC, SH>(si, s_st0, okm0, s_st3, okm3, s_st1);
                if (si + 1 >= steps) break;
                body.template operator()<VC, SH>(si + 1, s_st1, okm1, s_st0, okm0, s_st2);
                if (si + 2 >= steps) break;
                body.template operator()<VC, SH>(si + 2, s_st2, okm2, s_st1, okm1, s_st3);
                if (si + 3 >= steps) break;
                body.template operator()<VC, SH>(si + 3, s_st3, okm3, s_st2, okm2, s_st0);
            }
        }
        wait_vm<0>();  // no load may still be writing this workgroup's LDS when it ends
    };

    auto acc_finite = [&]() -> bool  // every accumulator of the wave is finite
    {
        float t = 0.0f;  // 0 if every accumulator is finite, else NaN
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) t = __builtin_fmaf(acc[gi][n][i], 0.0f, t);
        return !__any(!(t == 0.0f));
    };
    if constexpr (VCONV)
    {
        pipeline.template operator()<true, false>();
        if (!acc_finite()) s_vover = 1;
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();  // flags written; every wave is past its last reads of the stages
        if (s_vover != 0)              // uniform: some V value of the workgroup's keys does not fit f16
            pipeline.template operator()<false, false>();
    }
    else if constexpr (CT == I8)
    {
        // int8 pages: P carries the keys' V scales into the f16 PV products and p < 2^8, so a V scale of 256 or
        // more (a dequantized |V| from about 32,500) can overflow f16 and make the accumulators infinite or NaN.
        // The workgroup then runs the pipeline again with every p scaled by 2^-12, which takes V scales up to 2^20
        // (|V| up to about 1.3e8); products that the scaling takes below f16's normal range keep an absolute error
        // of at most 2^-13 of the unscaled p times the V scale.
        pipeline.template operator()<false, false>();
        if (!acc_finite()) s_vover = 1;
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();  // flags written; every wave is past its last reads of the stages
        if (s_vover != 0)              // uniform
            pipeline.template operator()<false, true>();
    }
    else
    {
        pipeline.template operator()<false, false>();
    }

#pragma unroll
    for (int gi = 0; gi < RG; ++gi)
    {
        const float l_tot = swap_sum(l_run[gi]) + lacc[gi][0];  // whichever of the two the pipeline filled
        if constexpr (PFX)
        {
            // partial of (row bq, head hq) over this chunk, in the decode merge's convention: max in the log2 domain
            if (col_ok[gi])
            {
                const int64_t slot =
                    static_cast<int64_t>(a.pfx_slot0) + static_cast<int64_t>(chunk) * a.batch + bq[gi];
                float* dst = a.ws_acc + (slot * Hq + hq[gi]) * D;
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    *reinterpret_cast<f32x4*>(dst + 16 * n + 4 * g) = acc[gi][n] * v_head_scale;
                if (g == 0)
                {
                    // (an int8 rerun scaled p by 2^kRerunShift, which the partial's max carries)
                    const float shift = CT == I8 && s_vover != 0 ? kRerunShift : 0.0f;
                    a.ws_ml[(slot * Hq + hq[gi]) * 2] = m_run[gi] == kNegInf ? kNegInf : m_run[gi] * c_log2 - shift;
                    a.ws_ml[(slot * Hq + hq[gi]) * 2 + 1] = l_tot;
                }
            }
        }
        else if (col_ok[gi])
        {
            const float  inv = l_tot > 0.0f ? v_head_scale / l_tot : 0.0f;
            const size_t ob = qrow[gi] * D;
#pragma unroll
            for (int n = 0; n < NT; ++n) store_out4<QT>(a.out, ob + 16 * n + 4 * g, acc[gi][n] * inv);
        }
    }
}

template <int QT, int D, int CT, bool PFX, int RG>
__global__ __launch_bounds__(512 / RG)
__attribute__((amdgpu_waves_per_eu(RG == 2 ? (D == 256 ? 1 : 2) : (D <= 128 ? (CT == I8 ? 3 : 4) : 1))))
void paged_prefill_dma(PrefillArgs a)
{
    using L = PrefillLds<QT, D, CT, PFX, RG>;
    __shared__ __align__(16) uint8_t s_st0[L::STAGE];
    __shared__ __align__(16) uint8_t s_st1[L::STAGE];
    __shared__ __align__(16) uint8_t s_st2[L::S2];
    __shared__ __align__(16) uint8_t s_st3[L::S3];
    __shared__ int s_vover;
    prefill_wg<QT, D, CT, PFX, RG>(a, static_cast<int>(blockIdx.x), s_st0, s_st1, s_st2, s_st3, s_vover);
}

#ifndef FFKV_DEVICE_BODIES_ONLY

namespace
{

template <int CT, int QT, bool PFX>
hipError_t launch_pfd_d(const PrefillArgs& a, hipStream_t stream)
{
    const int64_t rows = PFX ? static_cast<int64_t>(a.batch) * a.group : static_cast<int64_t>(a.seq_len) * a.group;
    const int64_t groups = PFX ? static_cast<int64_t>(a.num_kv_heads) * a.pfx_chunks
                               : static_cast<int64_t>(a.batch) * a.num_kv_heads;
    const int64_t nrb = (rows + kDmaRows - 1) / kDmaRows;
#if FFKV_PREFILL_XCD
    const int64_t wgs = (groups + kXcds - 1) / kXcds * kXcds * nrb;
#else
    const int64_t wgs = groups * nrb;
#endif
    if (wgs <= 0) return hipSuccess;
    if (wgs > INT32_MAX) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<unsigned>(wgs));
    // head_dim 256: one row group (two would not fit the registers).  Prefix partials: one row group, so their
    // few hundred workgroups still put two waves on every SIMD.
    constexpr int RG = PFX ? 1 : FFKV_PREFILL_RG;
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((paged_prefill_dma<QT, 64, CT, PFX, RG>), grid, dim3(512 / RG), 0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((paged_prefill_dma<QT, 128, CT, PFX, RG>), grid, dim3(512 / RG), 0, stream, a);
            break;
        default:
        {
            constexpr int RG256 = PFX ? 1 : FFKV_PREFILL_RG256;
            hipLaunchKernelGGL((paged_prefill_dma<QT, 256, CT, PFX, RG256>), grid, dim3(512 / RG256), 0, stream, a);
            break;
        }
    }
    return hipGetLastError();
}

template <int CT, bool PFX>
hipError_t launch_pfd_q(const PrefillArgs& a, hipStream_t stream)
{
    switch (a.qo_dtype)
    {
        case F32:
            return launch_pfd_d<CT, F32, PFX>(a, stream);
        case F16:
            return launch_pfd_d<CT, F16, PFX>(a, stream);
        default:
            return launch_pfd_d<CT, BF16, PFX>(a, stream);
    }
}

template <bool PFX>
hipError_t launch_pfd(const PrefillArgs& a, hipStream_t stream)
{
    // 8-bit caches read their scales in every workgroup (int8 per token, fp8 per head)
    if ((a.cache_dtype == I8 || a.cache_dtype == FP8) && (a.k_scale == nullptr || a.v_scale == nullptr))
        return hipErrorInvalidValue;
    switch (a.cache_dtype)
    {
        case F16:
            return launch_pfd_q<F16, PFX>(a, stream);
        case BF16:
            return launch_pfd_q<BF16, PFX>(a, stream);
        case I8:
            return launch_pfd_q<I8, PFX>(a, stream);
        default:
            return launch_pfd_q<FP8, PFX>(a, stream);
    }
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) { return launch_pfd<false>(a, stream); }

hipError_t launch_prefix_partials(const PrefillArgs& a, hipStream_t stream) { return launch_pfd<true>(a, stream); }

#endif  // FFKV_DEVICE_BODIES_ONLY

}  // namespace ffkv
