// paged_decode_pfx.hip - the shared-prefix decode's partials and the decode of the rows' own pages in one launch.
//
// ffkv_paged_decode_shared_prefix splits a decode whose rows share their first pages: the shared pages are
// attended once for all rows by the prefill kernel's prefix mode (a compute-bound workgroup per kv head, block of
// 128 query rows and chunk of pages), the rows' own pages by the split-K decode (bound by HBM), and a merge folds
// both.  Launched one after the other, the prefix partials run alone for their whole duration (about a fifth of
// the call on 120 rows over a 2048-token prefix) while HBM idles.  Here both run in one grid: the decode's work
// items 0 .. pfx_items - 1 (every head group of them) each compute one prefix task first and then their share of
// the rows' pages, which is smaller by pfx_share / 1024, while the other items stream pages from the start.
// Every workgroup holds the LDS of the larger of the two (the prefix stages); the V tiles of its decode reuse it.
//
// Taken for 16-bit caches at head_dim 128, where one decode workgroup and one prefix workgroup are both four waves
// of up to 256 registers (two workgroups per CU either way); other dtypes and head dims launch the two kernels.
#define FFKV_DEVICE_BODIES_ONLY 1
#include "paged_prefill_dma.hip"
#include "paged_decode_mfma.hip"
#undef FFKV_DEVICE_BODIES_ONLY

#include <cstdlib>

namespace ffkv
{

namespace
{

constexpr int kPfxD = 128;     // head_dim of the fused kernel
constexpr int kPfxWaves = 4;   // waves per workgroup: a decode head group, or a prefix row block (2 x 16 rows each)
constexpr int kPfxRG = 2;      // row groups per wave of the prefix part
static_assert(512 / kPfxRG == 64 * kPfxWaves, "prefix and decode workgroups are the same size");

// The fused grid needs decode workgroups of kPfxWaves waves (a build with other FFKV_MFMA_MAX_WAVES* values
// launches the two kernels instead).
template <int CT>
constexpr bool kPfxFits = kMfmaMaxWaves<CT, kPfxD> == kPfxWaves;

template <int CT, int QT>
struct PfxLds
{
    using L = PrefillLds<QT, kPfxD, CT, true, kPfxRG>;
    static constexpr int V = kPfxWaves * kBlockSize * kPfxD * 2;  // decode V tiles
    static constexpr int BYTES = L::BYTES > V ? L::BYTES : V;
};

// Workgroup (x, y): work item x of gridDim.x, head group y.  Items x < pfx_items first run prefix task
// (x / 8) * 8 * gridDim.y + y * 8 + x % 8 (tasks beyond the prefix's grid return at once): x % 8 is the XCD the
// workgroup runs on when gridDim.x is a multiple of 8, which keeps the prefill kernel's rule that a prefix chunk's
// row blocks share one XCD's L2.
template <int CT, int QT>
__global__ __launch_bounds__(64 * kPfxWaves) __attribute__((amdgpu_waves_per_eu(2, 8)))
void paged_decode_pfx(DecodeArgs a, PrefillArgs p)
{
    static_assert(kPfxFits<CT>, "decode workgroups of four waves");
    using L = typename PfxLds<CT, QT>::L;
    __shared__ __align__(16) uint8_t s_lds[PfxLds<CT, QT>::BYTES];
    __shared__ int s_vover;
    const int x = static_cast<int>(blockIdx.x);
    const int y = static_cast<int>(blockIdx.y);
    if (x < a.pfx_items)
    {
        const int task = (x >> 3) * 8 * static_cast<int>(gridDim.y) + y * 8 + (x & 7);
        prefill_wg<QT, kPfxD, CT, true, kPfxRG>(p, task, s_lds, s_lds + L::STAGE, s_lds + 2 * L::STAGE,
                                                 s_lds + 2 * L::STAGE + L::S2, s_vover);
        __syncthreads();  // every wave is past its last read of the stages before the V tiles reuse the LDS
    }
    decode_wg<CT, QT, kPfxD, true>(a, x, y, static_cast<int>(gridDim.x), kPfxWaves, reinterpret_cast<uint16_t*>(s_lds));
}

template <int CT, int QT>
const void* pfx_kernel()
{
    if constexpr (kPfxFits<CT>)
        return reinterpret_cast<const void*>(paged_decode_pfx<CT, QT>);
    else
        return nullptr;
}

const void* pfx_kernel_for(int cache_dtype, int qo_dtype)
{
    if (cache_dtype == BF16)
        return qo_dtype == F32 ? pfx_kernel<BF16, F32>() : (qo_dtype == F16 ? pfx_kernel<BF16, F16>() : pfx_kernel<BF16, BF16>());
    return qo_dtype == F32 ? pfx_kernel<F16, F32>() : (qo_dtype == F16 ? pfx_kernel<F16, F16>() : pfx_kernel<F16, BF16>());
}

template <int CT, int QT>
hipError_t launch_pfx(const DecodeArgs& a, const PrefillArgs& p, int gy, hipStream_t stream)
{
    if constexpr (kPfxFits<CT>)
    {
        hipLaunchKernelGGL((paged_decode_pfx<CT, QT>), dim3(static_cast<unsigned>(a.items), static_cast<unsigned>(gy)),
                           dim3(64 * kPfxWaves), 0, stream, a, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_merge<QT, kPfxD>(a, stream);
    }
    else
        return hipErrorInvalidConfiguration;  // not reached: decode_pfx_plan declines such builds
}

int env_int(const char* name, int dflt)
{
    const char* s = std::getenv(name);
    return s != nullptr && *s != '\0' ? std::atoi(s) : dflt;
}

}  // namespace

bool decode_pfx_plan(const DecodeArgs& a, int shared_pages, int max_chunks, DecodePfxPlan& plan)
{
    static const int fused_on = env_int("FFKV_PFX_FUSED", 1);
    if (fused_on == 0 || a.head_dim != kPfxD || (a.cache_dtype != BF16 && a.cache_dtype != F16) || a.group > 16 ||
        shared_pages <= 0 || max_chunks <= 0 || a.num_kv_heads % kPfxWaves != 0)
        return false;
    const void* kernel = pfx_kernel_for(a.cache_dtype, a.qo_dtype);
    if (kernel == nullptr) return false;
    const int gy = a.num_kv_heads / kPfxWaves;  // one wave per KV head (group <= 16), four per workgroup
    const int items = decode_mfma_items(kernel, 64 * kPfxWaves, gy);
    if (items < 8) return false;
    // Prefix tasks: (kv head, chunk of pages) groups, padded to whole rounds of 8 XCDs, times blocks of 128 query
    // rows.  About one task for every fourth workgroup of the grid, at most max_chunks chunks (the workspace's
    // prefix slots; FFKV_PREFIX_CHUNKS sets it).
    static const int env_chunks = env_int("FFKV_PREFIX_CHUNKS", 0);
    const int64_t nrb = (static_cast<int64_t>(a.batch) * a.group + 127) / 128;
    int64_t chunks = env_chunks > 0 ? max_chunks : (static_cast<int64_t>(items) * gy / 4) / (nrb * a.num_kv_heads);
    chunks = chunks > max_chunks ? max_chunks : (chunks < 1 ? 1 : chunks);
    plan.chunk_pages = static_cast<int>((shared_pages + chunks - 1) / chunks);
    plan.chunks = (shared_pages + plan.chunk_pages - 1) / plan.chunk_pages;
    const int64_t groups = static_cast<int64_t>(a.num_kv_heads) * plan.chunks;
    const int64_t tasks = (groups + 7) / 8 * 8 * nrb;
    const int64_t pfx_items = ((tasks + gy - 1) / gy + 7) / 8 * 8;
    if (pfx_items > items) return false;
    plan.items = items;
    plan.gy = gy;
    plan.pfx_items = static_cast<int>(pfx_items);
    static const int env_share = env_int("FFKV_PFX_SHARE", 0);
    plan.pfx_share = env_share > 0 && env_share <= 1024 ? env_share : kPfxDefaultShare;
    return true;
}

hipError_t launch_decode_pfx(const DecodeArgs& a, const PrefillArgs& p, int gy, hipStream_t stream)
{
    if (a.cache_dtype == BF16)
    {
        if (a.qo_dtype == F32) return launch_pfx<BF16, F32>(a, p, gy, stream);
        if (a.qo_dtype == F16) return launch_pfx<BF16, F16>(a, p, gy, stream);
        return launch_pfx<BF16, BF16>(a, p, gy, stream);
    }
    if (a.qo_dtype == F32) return launch_pfx<F16, F32>(a, p, gy, stream);
    if (a.qo_dtype == F16) return launch_pfx<F16, F16>(a, p, gy, stream);
    return launch_pfx<F16, BF16>(a, p, gy, stream);
}

}  // namespace ffkv
