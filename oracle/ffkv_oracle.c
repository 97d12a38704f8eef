/*
 * ffkv_oracle.c - CPU restatement of Firefly's paged KV-cache path (append + PagedAttention decode).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and bench.py's CPU baseline; never linked into or
 * called by the product library.
 *
 * Followed reference code (paths relative to the reference repository):
 *   append   src/model/qwen_model.cu:21-47    pos = ctx + t, page = table[b*max_blocks + pos/16], slot = pos%16,
 *                                            dst = ((page*16 + slot)*Hkv + h)*D + d, src = ((b*S + t)*Hkv + h)*D + d
 *   decode   src/kernels/attention.cu:291-447 context = ctx + 1 (:320), tail block holds context%16 or 16 tokens
 *                                            (:335-336), kv_head = h / (Hq/Hkv) (:304), eight token groups
 *                                            (tx/16, :307-309) each with an fp32 online softmax seeded at -1e30
 *                                            (:323-325, :372-399), 8-lane-chunk dot plus a 16-lane shuffle tree
 *                                            (:345-369), final merge of the eight states (:403-446)
 *   dispatch src/kernels/attention.cu:455-458 scale = 1/sqrtf(head_dim)
 *   rope     src/kernels/rope.cu:22-137       rotate-half pairs (i, i + D/2), pos = ctx + t, theta^(-2i/D)
 *   prefill  src/kernels/attention.cu:22-286  causal attention (key n > query m masked, :173-174), generalized
 *                                            to queries at ctx + t over the paged cache (prefix included)
 *
 * Extensions the reference does not have (it is fp16-only and leaves bad addressing undefined), restated
 * from the specification in include/ffkv.h: bf16/fp32 storage, int8 and OCP fp8 e4m3 quantization, skipped
 * writes and masked reads for invalid pages, zero output for rows without a valid token.
 *
 * Build: -O3 -march=native -ffp-contract=off.  Multiply-adds that nvcc contracts in the reference kernel are
 * written as explicit fmaf() calls; nothing else is contracted.
 *
 * Parity status of each function (what pins it; the tests live in tests/test_oracle.py):
 *   conversions   bf16/f16: exhaustive round trip + numpy/torch RNE on random and tie inputs;
 *                 e4m3: all 256 codes round-trip, midpoints round to even, torch float8_e4m3fn for |x| <= 448,
 *                 saturation edge pinned by the OCP spec values (448, 464, inf, NaN).
 *   int8 quant    torch.round (half-even) on the closed form, golden fixtures.
 *   ffo_append    closed-form address formula in numpy, whole-pool sentinel check, append->gather round trip.
 *   ffo_paged_prefill_f64  seq_len = 1 equals ffo_paged_decode_f64; torch SDPA with an explicit causal mask on
 *                 the gathered K/V (prefix included); contiguous mode = torch SDPA is_causal; shared prefix
 *                 = private copy.
 *   ffo_rope      torch float64 rotate_half formulation (q*cos + rotate_half(q)*sin), position 0 = identity,
 *                 unit vectors give (cos, sin), pair norms preserved, q.k depends only on the position offset.
 *   ffo_paged_decode  float64 closed form (ffo_paged_decode_f64), torch SDPA on gathered K/V with repeated
 *                 heads, special cases (one token, constant K, dominant logit, GQA symmetry, shared prefix).
 */
#define _GNU_SOURCE
#include "ffkv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define DT_F32 0
#define DT_F16 1
#define DT_BF16 2
#define DT_I8 3
#define DT_FP8 8

#define ERR_ARG -1
#define ERR_UNSUPPORTED -2

static inline uint32_t f2u(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

static inline float u2f(uint32_t u)
{
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* ----------------------------------------------------------------------------------------------------------
 * Scalar conversions, all round-to-nearest-even.
 * -------------------------------------------------------------------------------------------------------- */

uint16_t ffo_f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float ffo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t ffo_f32_to_f16(float x)
{
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;  /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (a < 0x38800000u)                         /* below 2^-14: subnormal half, code = rne(|x| * 2^24) */
        return sign | (uint16_t)rintf(u2f(a) * 16777216.0f);
    a += 0xfffu + ((a >> 13) & 1u);
    a -= 112u << 23;
    return sign | (uint16_t)(a >> 13);
}

float ffo_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) return u2f(sign) + (sign ? -1.0f : 1.0f) * ldexpf((float)m, -24);
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint8_t ffo_f32_to_e4m3(float x)
{
    uint32_t u = f2u(x);
    uint8_t  sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;  /* NaN */
    if (a >= 0x43e00000u) return sign | 0x7eu; /* |x| >= 448 (incl. inf): saturate to 448 */
    if (a < 0x3c800000u)                       /* |x| < 2^-6: subnormal, code = rne(|x| * 2^9) in 0..8 */
        return sign | (uint8_t)rintf(u2f(a) * 512.0f);
    a += 0x7ffffu + ((a >> 20) & 1u); /* round the 23-bit mantissa to 3 bits, carry into the exponent */
    uint32_t code = (a >> 20) - (120u << 3);
    if (code > 0x7eu) code = 0x7eu;
    return sign | (uint8_t)code;
}

float ffo_e4m3_to_f32(uint8_t q)
{
    uint32_t mag = q & 0x7fu;
    float    v;
    if (mag == 0x7fu)
        v = NAN;
    else if ((mag >> 3) == 0)
        v = ldexpf((float)(mag & 7u), -9);
    else
        v = ldexpf(1.0f + (float)(mag & 7u) / 8.0f, (int)(mag >> 3) - 7);
    return (q & 0x80u) ? -v : v;
}

float ffo_quant_i8_row(const float* x, int n, int8_t* q)
{
    float amax = 0.0f;
    for (int i = 0; i < n; ++i)
    {
        float a = fabsf(x[i]);
        if (a > amax) amax = a; /* NaN never compares greater: ignored */
    }
    if (amax == 0.0f)
    {
        memset(q, 0, (size_t)n);
        return 0.0f;
    }
    float s = amax / 127.0f;
    for (int i = 0; i < n; ++i)
    {
        float y = x[i] / s;
        if (isnan(y))
        {
            q[i] = 0;
            continue;
        }
        float r = rintf(y);
        if (r > 127.0f) r = 127.0f;
        if (r < -127.0f) r = -127.0f;
        q[i] = (int8_t)r;
    }
    return s;
}

void ffo_cvt_f32_to_bf16(const float* x, uint16_t* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_f32_to_bf16(x[i]);
}
void ffo_cvt_f32_to_f16(const float* x, uint16_t* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_f32_to_f16(x[i]);
}
void ffo_cvt_f32_to_e4m3(const float* x, uint8_t* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_f32_to_e4m3(x[i]);
}
void ffo_cvt_e4m3_to_f32(const uint8_t* x, float* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_e4m3_to_f32(x[i]);
}
void ffo_cvt_bf16_to_f32(const uint16_t* x, float* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_bf16_to_f32(x[i]);
}
void ffo_cvt_f16_to_f32(const uint16_t* x, float* y, size_t n)
{
    for (size_t i = 0; i < n; ++i) y[i] = ffo_f16_to_f32(x[i]);
}

/* ----------------------------------------------------------------------------------------------------------
 * Element access helpers.
 * -------------------------------------------------------------------------------------------------------- */

static int is_act_dtype(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16; }
static int is_cache_dtype(int dt) { return is_act_dtype(dt) || dt == DT_I8 || dt == DT_FP8; }

static size_t dtype_bytes(int dt)
{
    switch (dt)
    {
        case DT_F32:
            return 4;
        case DT_F16:
        case DT_BF16:
            return 2;
        default:
            return 1;
    }
}

static inline float load_act(const void* p, int dt, size_t i)
{
    switch (dt)
    {
        case DT_F32:
            return ((const float*)p)[i];
        case DT_F16:
            return ffo_f16_to_f32(((const uint16_t*)p)[i]);
        default:
            return ffo_bf16_to_f32(((const uint16_t*)p)[i]);
    }
}

static inline void store_act(void* p, int dt, size_t i, float x)
{
    switch (dt)
    {
        case DT_F32:
            ((float*)p)[i] = x;
            break;
        case DT_F16:
            ((uint16_t*)p)[i] = ffo_f32_to_f16(x);
            break;
        default:
            ((uint16_t*)p)[i] = ffo_f32_to_bf16(x);
            break;
    }
}

/* Dequantized value of cache element `idx` (element index into [N,16,Hkv,D]); `srow` is the (page,slot,head)
 * row index used by int8 scales and `h` the kv head used by fp8 scales. */
static inline float load_cache(const void* c, int dt, size_t idx, const float* scale, size_t srow, int h)
{
    switch (dt)
    {
        case DT_I8:
            return (float)((const int8_t*)c)[idx] * scale[srow];
        case DT_FP8:
            return ffo_e4m3_to_f32(((const uint8_t*)c)[idx]) * scale[h];
        default:
            return load_act(c, dt, idx);
    }
}

/* ----------------------------------------------------------------------------------------------------------
 * Append.  Restates src/model/qwen_model.cu:21-47 (one thread per element d of (t, h, b)).
 * -------------------------------------------------------------------------------------------------------- */

static void append_one(const void* src, int sdt, void* cache, int cdt, float* scale, size_t src_row, size_t dst_row,
                       size_t srow, int h, int D, float* tmp, int8_t* qtmp)
{
    size_t s0 = src_row * (size_t)D, d0 = dst_row * (size_t)D;
    if (sdt == cdt && cdt != DT_I8 && cdt != DT_FP8)
    {
        size_t b = dtype_bytes(cdt);
        memcpy((char*)cache + d0 * b, (const char*)src + s0 * b, (size_t)D * b);
        return;
    }
    for (int d = 0; d < D; ++d) tmp[d] = load_act(src, sdt, s0 + d);
    if (cdt == DT_I8)
    {
        scale[srow] = ffo_quant_i8_row(tmp, D, qtmp);
        memcpy((int8_t*)cache + d0, qtmp, (size_t)D);
    }
    else if (cdt == DT_FP8)
    {
        float s = scale[h];
        for (int d = 0; d < D; ++d) ((uint8_t*)cache)[d0 + d] = ffo_f32_to_e4m3(tmp[d] / s);
    }
    else
    {
        for (int d = 0; d < D; ++d) store_act(cache, cdt, d0 + d, tmp[d]);
    }
}

typedef struct
{
    const void *k_src, *v_src;
    void *      k_cache, *v_cache;
    float *     k_scale, *v_scale;
    const int32_t* block_table;
    const int32_t* context_lens;
    int src_dtype, cache_dtype, batch, seq_len, num_kv_heads, head_dim, max_blocks, num_blocks;
    int h0, h1; /* kv heads of this worker */
} append_job;

/* Heads h0 .. h1-1 of every token.  Each head owns disjoint bytes of the pages and its own int8 scales, so
 * workers over disjoint head ranges write disjoint memory, and within a head the (b, t) order is the serial one
 * (the last writer of a slot shared by two rows' tables wins, as in a serial run). */
static void* append_worker(void* arg)
{
    const append_job* j = (const append_job*)arg;
    float*            tmp = (float*)malloc(sizeof(float) * (size_t)j->head_dim);
    int8_t*           qtmp = (int8_t*)malloc((size_t)j->head_dim);
    for (int b = 0; b < j->batch; ++b)
    {
        int ctx0 = j->context_lens ? j->context_lens[b] : 0; /* qwen_model.cu:32 */
        for (int t = 0; t < j->seq_len; ++t)
        {
            long long pos = (long long)ctx0 + t; /* :33 */
            if (pos < 0) continue;
            long long blk = pos / 16, off = pos % 16; /* :34-35 */
            if (blk >= j->max_blocks) continue;
            int phys = j->block_table[(size_t)b * (size_t)j->max_blocks + (size_t)blk]; /* :37 */
            if (phys < 0 || phys >= j->num_blocks) continue;
            for (int h = j->h0; h < j->h1; ++h)
            {
                size_t src_row = ((size_t)b * j->seq_len + t) * j->num_kv_heads + h;                /* :39 */
                size_t dst_row = ((size_t)phys * 16 + (size_t)off) * j->num_kv_heads + (size_t)h; /* :41-42 */
                append_one(j->k_src, j->src_dtype, j->k_cache, j->cache_dtype, j->k_scale, src_row, dst_row, dst_row,
                           h, j->head_dim, tmp, qtmp);
                append_one(j->v_src, j->src_dtype, j->v_cache, j->cache_dtype, j->v_scale, src_row, dst_row, dst_row,
                           h, j->head_dim, tmp, qtmp);
            }
        }
    }
    free(tmp);
    free(qtmp);
    return NULL;
}

int ffo_append(const void* k_src, const void* v_src, int src_dtype, void* k_cache, void* v_cache, int cache_dtype,
               float* k_scale, float* v_scale, const int32_t* block_table, const int32_t* context_lens, int batch,
               int seq_len, int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_blocks)
{
    if (block_size != 16) return ERR_UNSUPPORTED;
    if (!is_act_dtype(src_dtype) || !is_cache_dtype(cache_dtype)) return ERR_UNSUPPORTED;
    if (batch < 0 || seq_len < 0 || num_kv_heads <= 0 || head_dim <= 0 || max_blocks < 0 || num_blocks < 0)
        return ERR_ARG;
    if (batch == 0 || seq_len == 0) return 0;
    if (!k_src || !v_src || !k_cache || !v_cache || !block_table) return ERR_ARG;
    if ((cache_dtype == DT_I8 || cache_dtype == DT_FP8) && (!k_scale || !v_scale)) return ERR_ARG;

    append_job base = {k_src,      v_src,       k_cache,   v_cache,     k_scale,  v_scale,
                       block_table, context_lens, src_dtype, cache_dtype, batch,    seq_len,
                       num_kv_heads, head_dim,    max_blocks, num_blocks, 0,        num_kv_heads};
    /* large appends run one worker per group of kv heads (the result does not depend on the split) */
    int workers = (long long)batch * seq_len >= 4096 ? ffo_default_threads() : 1;
    if (workers > num_kv_heads) workers = num_kv_heads;
    if (workers <= 1)
    {
        append_worker(&base);
        return 0;
    }
    append_job* jobs = (append_job*)malloc(sizeof(append_job) * (size_t)workers);
    pthread_t*  tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)workers);
    for (int i = 0; i < workers; ++i)
    {
        jobs[i] = base;
        jobs[i].h0 = (int)((long long)num_kv_heads * i / workers);
        jobs[i].h1 = (int)((long long)num_kv_heads * (i + 1) / workers);
        pthread_create(&tids[i], NULL, append_worker, &jobs[i]);
    }
    for (int i = 0; i < workers; ++i) pthread_join(tids[i], NULL);
    free(tids);
    free(jobs);
    return 0;
}

/* ----------------------------------------------------------------------------------------------------------
 * Rotary embedding.  Restates rope_kernel_optimized (src/kernels/rope.cu:22-137): position pos = ctx[b] + t
 * (t when ctx is null, :36-37), pair i = (dims i, i + D/2) rotated by pos * theta^(-2i/D) (:74-77) in the
 * rotate-half form lo' = lo*c - hi*s, hi' = hi*c + lo*s (:84-91), written back in the tensor's dtype.  The
 * arithmetic is the one include/ffkv.h specifies (the reference's fast-math powf/cosf/sinf are not
 * reproducible): inv_freq, cos and sin in double rounded once to float, the angle one float product, the
 * rotation float products and sums (built with -ffp-contract=off, so each is rounded separately).
 * -------------------------------------------------------------------------------------------------------- */

int ffo_rope(void* x, int dtype, const int32_t* context_lens, int batch, int seq_len, int heads, int head_dim,
             float theta)
{
    if (!is_act_dtype(dtype)) return ERR_UNSUPPORTED;
    if (batch < 0 || seq_len < 0 || heads < 0 || head_dim <= 0 || (head_dim & 1)) return ERR_ARG;
    if (!(theta > 0.0f)) return ERR_ARG;
    if (batch == 0 || seq_len == 0 || heads == 0) return 0;
    if (!x) return ERR_ARG;
    const int half = head_dim / 2;
    float*    cs = (float*)malloc(sizeof(float) * 2 * (size_t)half);
    for (int b = 0; b < batch; ++b)
    {
        for (int t = 0; t < seq_len; ++t)
        {
            long long pos = (long long)(context_lens ? context_lens[b] : 0) + t; /* rope.cu:36-37 */
            for (int i = 0; i < half; ++i)
            {
                float inv_freq = (float)pow((double)theta, -2.0 * i / head_dim); /* :74-76 */
                float ang = (float)pos * inv_freq;                              /* :77 */
                cs[2 * i] = (float)cos((double)ang);
                cs[2 * i + 1] = (float)sin((double)ang);
            }
            for (int h = 0; h < heads; ++h)
            {
                size_t base = (((size_t)b * seq_len + t) * heads + h) * (size_t)head_dim;
                for (int i = 0; i < half; ++i)
                {
                    float c = cs[2 * i], s = cs[2 * i + 1];
                    float lo = load_act(x, dtype, base + i), hi = load_act(x, dtype, base + i + half);
                    float lc = lo * c, hs = hi * s, hc = hi * c, ls = lo * s;
                    store_act(x, dtype, base + i, lc - hs);   /* :84-85 */
                    store_act(x, dtype, base + i + half, hc + ls);
                }
            }
        }
    }
    free(cs);
    return 0;
}

/* ----------------------------------------------------------------------------------------------------------
 * Decode.  Restates paged_attention_kernel (src/kernels/attention.cu:291-447) for one (sequence, head).
 * -------------------------------------------------------------------------------------------------------- */

typedef struct
{
    const void*    q;
    void*          out;
    int            qo_dtype;
    const void*    k_cache;
    const void*    v_cache;
    int            cache_dtype;
    const float*   k_scale;
    const float*   v_scale;
    const int32_t* block_table;
    const int32_t* context_lens;
    int            batch, num_heads, num_kv_heads, head_dim, max_blocks, num_blocks, max_context_len;
    float          scale;
    float*         out_f32;
    atomic_int     next;
} decode_job;

/* Attended token count of row b after the +1 of src/kernels/attention.cu:320 and the documented clamps. */
static long long row_context(const int32_t* ctx, int b, int max_blocks, int max_context_len)
{
    long long L = (long long)ctx[b] + 1;
    long long cap = (long long)max_blocks * 16;
    if (max_context_len > 0 && cap > max_context_len) cap = max_context_len;
    if (L > cap) L = cap;
    return L < 0 ? 0 : L;
}

static void decode_row(decode_job* j, int b, int h, float* qv, float* acc, float* part, float* kv)
{
    const int D = j->head_dim;
    const int kvh = h / (j->num_heads / j->num_kv_heads); /* :304 */
    const size_t qoff = ((size_t)b * j->num_heads + (size_t)h) * (size_t)D;
    for (int d = 0; d < D; ++d) qv[d] = load_act(j->q, j->qo_dtype, qoff + d);

    const int lanes = (D + 7) / 8; /* 16-B lanes per token: 16 for D = 128 (:309) */
    int       tree = 1;
    while (tree < lanes) tree <<= 1;

    float m[8], l[8];
    for (int g = 0; g < 8; ++g)
    {
        m[g] = -1e30f; /* :323 */
        l[g] = 0.0f;
    }
    memset(acc, 0, sizeof(float) * 8 * (size_t)D);

    long long L = row_context(j->context_lens, b, j->max_blocks, j->max_context_len);
    long long nblk = (L + 15) / 16; /* :321 */
    for (long long blk = 0; blk < nblk; ++blk)
    {
        int  phys = j->block_table[(size_t)b * (size_t)j->max_blocks + (size_t)blk]; /* :334 */
        int  page_ok = phys >= 0 && phys < j->num_blocks;
        int  tib = (blk == nblk - 1) ? (int)(L % 16) : 16; /* :335-336 */
        if (tib == 0) tib = 16;
        for (int t0 = 0; t0 < tib; t0 += 8) /* :338 */
        {
            for (int g = 0; g < 8; ++g)
            {
                int   t = t0 + g; /* :340 */
                int   valid = t < tib && page_ok;
                float score = -1e30f;
                if (valid)
                {
                    size_t row = ((size_t)phys * 16 + (size_t)t) * j->num_kv_heads + (size_t)kvh; /* :347-348 */
                    size_t base = row * (size_t)D;
                    for (int d = 0; d < D; ++d)
                        kv[d] = load_cache(j->k_cache, j->cache_dtype, base + d, j->k_scale, row, kvh);
                    for (int v = 0; v < tree; ++v)
                    {
                        float s = 0.0f;
                        for (int i = 0; i < 8 && v * 8 + i < D && v < lanes; ++i)
                            s = fmaf(qv[v * 8 + i], kv[v * 8 + i], s); /* :354-357 */
                        part[v] = s;
                    }
                    for (int off = tree / 2; off > 0; off /= 2) /* shuffle tree, :363-366 */
                        for (int v = 0; v < off; ++v) part[v] += part[v + off];
                    score = part[0] * j->scale; /* :369 */
                }
                float m_prev = m[g]; /* :373-379 */
                m[g] = fmaxf(m[g], score);
                float alpha = valid ? expf(score - m[g]) : 0.0f;
                float beta = expf(m_prev - m[g]);
                l[g] = fmaf(l[g], beta, alpha);
                float* a = acc + (size_t)g * D;
                for (int d = 0; d < D; ++d) a[d] *= beta; /* :382-385 */
                if (valid)
                {
                    size_t row = ((size_t)phys * 16 + (size_t)t) * j->num_kv_heads + (size_t)kvh;
                    size_t base = row * (size_t)D;
                    for (int d = 0; d < D; ++d)
                        a[d] = fmaf(load_cache(j->v_cache, j->cache_dtype, base + d, j->v_scale, row, kvh), alpha,
                                    a[d]); /* :391-398 */
                }
            }
        }
    }

    /* merge of the eight group states, :418-441 */
    float fm = -1e30f, fl = 0.0f;
    for (int g = 0; g < 8; ++g) fm = fmaxf(fm, m[g]);
    float w[8];
    for (int g = 0; g < 8; ++g)
    {
        w[g] = expf(m[g] - fm);
        fl = fmaf(l[g], w[g], fl);
    }
    for (int d = 0; d < D; ++d)
    {
        float fa = 0.0f;
        for (int g = 0; g < 8; ++g) fa = fmaf(acc[(size_t)g * D + d], w[g], fa);
        float o = fl > 0.0f ? fa / fl : 0.0f; /* :445; zero when no token was valid */
        store_act(j->out, j->qo_dtype, qoff + d, o);
        if (j->out_f32) j->out_f32[qoff + d] = o;
    }
}

static void* decode_worker(void* arg)
{
    decode_job* j = (decode_job*)arg;
    int         D = j->head_dim;
    float*      qv = (float*)malloc(sizeof(float) * (size_t)D);
    float*      acc = (float*)malloc(sizeof(float) * 8 * (size_t)D);
    float*      part = (float*)malloc(sizeof(float) * 64);
    float*      kv = (float*)malloc(sizeof(float) * (size_t)D);
    int         total = j->batch * j->num_heads;
    for (;;)
    {
        int item = atomic_fetch_add(&j->next, 1);
        if (item >= total) break;
        decode_row(j, item / j->num_heads, item % j->num_heads, qv, acc, part, kv);
    }
    free(qv);
    free(acc);
    free(part);
    free(kv);
    return NULL;
}

/* Worker threads: the CPUs this process may run on (its affinity mask), at most 16 (a GPU box's host share). */
int ffo_default_threads(void)
{
    cpu_set_t set;
    long      n = sched_getaffinity(0, sizeof(set), &set) == 0 ? CPU_COUNT(&set) : sysconf(_SC_NPROCESSORS_ONLN);
    if (n > 16) n = 16;
    return n > 0 ? (int)n : 1;
}

static int check_decode_args(const void* q, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                             const float* k_scale, const float* v_scale, const int32_t* block_table,
                             const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                             int block_size, int max_blocks, int num_blocks)
{
    if (block_size != 16) return ERR_UNSUPPORTED;
    if (!is_act_dtype(qo_dtype) || !is_cache_dtype(cache_dtype)) return ERR_UNSUPPORTED;
    if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim > 512 || max_blocks < 0 ||
        num_blocks < 0)
        return ERR_ARG;
    if (num_heads % num_kv_heads != 0) return ERR_ARG;
    if (batch == 0) return 0;
    if (!q || !k_cache || !v_cache || !block_table || !context_lens) return ERR_ARG;
    if ((cache_dtype == DT_I8 || cache_dtype == DT_FP8) && (!k_scale || !v_scale)) return ERR_ARG;
    return 1;
}

int ffo_paged_decode(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                     int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                     const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                     int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                     float* out_f32, int threads)
{
    int rc = check_decode_args(q, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table,
                               context_lens, batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks,
                               num_blocks);
    if (rc <= 0) return rc;
    if (!out) return ERR_ARG;

    decode_job j = {q,          out,        qo_dtype,     k_cache,  v_cache,    cache_dtype,
                    k_scale,    v_scale,    block_table,  context_lens, batch,    num_heads,
                    num_kv_heads, head_dim, max_blocks,   num_blocks, max_context_len,
                    scale > 0.0f ? scale : 1.0f / sqrtf((float)head_dim), out_f32, 0};
    atomic_init(&j.next, 0);

    if (threads <= 0) threads = ffo_default_threads();
    if (threads > batch * num_heads) threads = batch * num_heads;
    if (threads <= 1)
    {
        decode_worker(&j);
        return 0;
    }
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, decode_worker, &j);
    for (int i = 0; i < threads; ++i) pthread_join(tids[i], NULL);
    free(tids);
    return 0;
}

int ffo_paged_decode_f64(const void* q, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                         const float* k_scale, const float* v_scale, const int32_t* block_table,
                         const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                         int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                         double* out)
{
    int rc = check_decode_args(q, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table,
                               context_lens, batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks,
                               num_blocks);
    if (rc <= 0) return rc;
    if (!out) return ERR_ARG;
    const int    D = head_dim;
    const double sc = scale > 0.0f ? (double)scale : 1.0 / sqrt((double)head_dim);
    const int    G = num_heads / num_kv_heads;

    for (int b = 0; b < batch; ++b)
    {
        long long L = row_context(context_lens, b, max_blocks, max_context_len);
        double*   s = (double*)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
        long long* rows = (long long*)malloc(sizeof(long long) * (size_t)(L > 0 ? L : 1));
        for (int h = 0; h < num_heads; ++h)
        {
            int     kvh = h / G;
            double* o = out + ((size_t)b * num_heads + (size_t)h) * (size_t)D;
            size_t  qoff = ((size_t)b * num_heads + (size_t)h) * (size_t)D;
            long long n = 0;
            double  mx = -INFINITY;
            for (long long t = 0; t < L; ++t)
            {
                int phys = block_table[(size_t)b * (size_t)max_blocks + (size_t)(t / 16)];
                if (phys < 0 || phys >= num_blocks) continue;
                long long row = ((long long)phys * 16 + t % 16) * num_kv_heads + kvh;
                double    dot = 0.0;
                for (int d = 0; d < D; ++d)
                    dot += (double)load_act(q, qo_dtype, qoff + d) *
                           (double)load_cache(k_cache, cache_dtype, (size_t)row * D + d, k_scale, (size_t)row, kvh);
                s[n] = dot * sc;
                rows[n] = row;
                if (s[n] > mx) mx = s[n];
                ++n;
            }
            for (int d = 0; d < D; ++d) o[d] = 0.0;
            if (n == 0) continue;
            double den = 0.0;
            for (long long i = 0; i < n; ++i)
            {
                double p = exp(s[i] - mx);
                den += p;
                for (int d = 0; d < D; ++d)
                    o[d] += p * (double)load_cache(v_cache, cache_dtype, (size_t)rows[i] * D + d, v_scale,
                                                   (size_t)rows[i], kvh);
            }
            for (int d = 0; d < D; ++d) o[d] /= den;
        }
        free(s);
        free(rows);
    }
    return 0;
}

/* ----------------------------------------------------------------------------------------------------------
 * Prefill (chunked, paged).  Extends the decode restatement to seq_len query tokens per row: query t of row b
 * sits at position ctx[b] + t and attends the keys 0 .. ctx[b] + t of the row (causal over the cached prefix and
 * the chunk), read after this chunk's K/V were appended; keys at or beyond L_b = ctx[b] + seq_len (clamped to
 * [0, max_blocks*16] and to max_context_len > 0) or on an invalid page are skipped.  With block_table == NULL
 * the K/V are contiguous [batch, seq_len, Hkv, D] and ctx is 0: the causal attention of the reference's prefill
 * branch (flash_attn_wmma_kernel, src/kernels/attention.cu:22-286, key n masked when n >= seq_len or n > m at
 * :173-174, scale 1/sqrtf(D) at :458).  With seq_len = 1 it equals ffo_paged_decode_f64.  Closed form in
 * float64; out is [batch, seq_len, num_heads, head_dim].  The (row, query token) items run on worker threads;
 * each item's arithmetic does not depend on the thread count.
 * -------------------------------------------------------------------------------------------------------- */

typedef struct
{
    const void *q, *k_cache, *v_cache;
    int qo_dtype, cache_dtype;
    const float *k_scale, *v_scale;
    const int32_t *block_table, *context_lens;
    int batch, seq_len, num_heads, num_kv_heads, head_dim, max_blocks, num_blocks;
    long long cap, max_keys;
    double sc;
    double* out;
    atomic_int next;
} prefill_job;

enum { PREFILL_TOKENS_PER_ITEM = 32 };

typedef struct
{
    double *kt, *kraw, *v, *s, *qd;
    long long* pos;
} prefill_scratch;

/* One item: query tokens [t0, t1) of row b against kv head kvh, for the kv head's G query heads.  The row's keys
 * (those on valid pages below the row's limit) are read once into float64 K^T [D][n] and V [n][D]; key k's
 * score is the sum over d in increasing order of q[d]*K[k][d], so vectorising across keys keeps that order. */
static void prefill_item(const prefill_job* j, int b, int kvh, int t0, int t1, prefill_scratch* w)
{
    const int D = j->head_dim, S = j->seq_len, H = j->num_heads, G = j->num_heads / j->num_kv_heads;
    const int paged = j->block_table != NULL;
    long long ctx = paged ? (long long)j->context_lens[b] : 0;
    long long L = ctx + S;
    if (paged && L > j->cap) L = j->cap;
    if (L < 0) L = 0;
    long long kmax = ctx + t1;  /* keys any query of the item may see */
    if (kmax > L) kmax = L;
    long long nk = 0;
    for (long long k = 0; k < kmax; ++k)
    {
        long long row;
        if (paged)
        {
            int phys = j->block_table[(size_t)b * (size_t)j->max_blocks + (size_t)(k / 16)];
            if (phys < 0 || phys >= j->num_blocks) continue;
            row = ((long long)phys * 16 + k % 16) * j->num_kv_heads + kvh;
        }
        else
        {
            row = ((long long)b * S + k) * j->num_kv_heads + kvh;
        }
        w->pos[nk++] = k;
        for (int d = 0; d < D; ++d)
        {
            w->v[(size_t)(nk - 1) * (size_t)D + d] =
                (double)load_cache(j->v_cache, j->cache_dtype, (size_t)row * D + d, j->v_scale, (size_t)row, kvh);
            w->kraw[(size_t)(nk - 1) * (size_t)D + d] =
                (double)load_cache(j->k_cache, j->cache_dtype, (size_t)row * D + d, j->k_scale, (size_t)row, kvh);
        }
    }
    for (long long i = 0; i < nk; ++i)  /* K^T with row stride nk */
        for (int d = 0; d < D; ++d) w->kt[(size_t)d * (size_t)nk + (size_t)i] = w->kraw[(size_t)i * (size_t)D + d];
    for (int t = t0; t < t1; ++t)
    {
        long long kend = ctx + t + 1;  /* keys at positions < kend are visible */
        long long m = 0;               /* visible keys: a prefix of the item's key list (positions increase) */
        while (m < nk && w->pos[m] < kend) ++m;
        for (int g = 0; g < G; ++g)
        {
            const int h = kvh * G + g;
            double*   o = j->out + (((size_t)b * S + t) * H + (size_t)h) * (size_t)D;
            size_t    qoff = (((size_t)b * S + t) * H + (size_t)h) * (size_t)D;
            for (int d = 0; d < D; ++d) o[d] = 0.0;
            if (m == 0) continue;
            for (int d = 0; d < D; ++d) w->qd[d] = (double)load_act(j->q, j->qo_dtype, qoff + d);
            double* s = w->s;
            for (long long i = 0; i < m; ++i) s[i] = 0.0;
            for (int d = 0; d < D; ++d)
            {
                const double  qv = w->qd[d];
                const double* kr = w->kt + (size_t)d * (size_t)nk;
                for (long long i = 0; i < m; ++i) s[i] += qv * kr[i];
            }
            double mx = -INFINITY;
            for (long long i = 0; i < m; ++i)
            {
                s[i] *= j->sc;
                if (s[i] > mx) mx = s[i];
            }
            double den = 0.0;
            for (long long i = 0; i < m; ++i)
            {
                double p = exp(s[i] - mx);
                den += p;
                const double* vr = w->v + (size_t)i * (size_t)D;
                for (int d = 0; d < D; ++d) o[d] += p * vr[d];
            }
            for (int d = 0; d < D; ++d) o[d] /= den;
        }
    }
}

static void* prefill_worker(void* arg)
{
    prefill_job*    j = (prefill_job*)arg;
    size_t          nk = (size_t)(j->max_keys > 0 ? j->max_keys : 1);
    size_t          D = (size_t)j->head_dim;
    prefill_scratch w = {(double*)malloc(sizeof(double) * nk * D), (double*)malloc(sizeof(double) * nk * D),
                         (double*)malloc(sizeof(double) * nk * D), (double*)malloc(sizeof(double) * nk),
                         (double*)malloc(sizeof(double) * D), (long long*)malloc(sizeof(long long) * nk)};
    const int chunks = (j->seq_len + PREFILL_TOKENS_PER_ITEM - 1) / PREFILL_TOKENS_PER_ITEM;
    const int total = j->batch * j->num_kv_heads * chunks;
    for (;;)
    {
        int item = atomic_fetch_add(&j->next, 1);
        if (item >= total) break;
        int c = item % chunks, r = item / chunks;
        int t0 = c * PREFILL_TOKENS_PER_ITEM, t1 = t0 + PREFILL_TOKENS_PER_ITEM;
        if (t1 > j->seq_len) t1 = j->seq_len;
        prefill_item(j, r / j->num_kv_heads, r % j->num_kv_heads, t0, t1, &w);
    }
    free(w.kt);
    free(w.kraw);
    free(w.v);
    free(w.s);
    free(w.qd);
    free(w.pos);
    return NULL;
}

int ffo_paged_prefill_f64(const void* q, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                          const float* k_scale, const float* v_scale, const int32_t* block_table,
                          const int32_t* context_lens, int batch, int seq_len, int num_heads, int num_kv_heads,
                          int head_dim, int max_blocks, int num_blocks, int max_context_len, float scale, double* out)
{
    if (!is_act_dtype(qo_dtype) || !is_cache_dtype(cache_dtype)) return ERR_UNSUPPORTED;
    if (batch < 0 || seq_len < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        num_heads % num_kv_heads != 0 || max_blocks < 0 || num_blocks < 0)
        return ERR_ARG;
    if (batch == 0 || seq_len == 0) return 0;
    const int paged = block_table != NULL;
    if (!q || !k_cache || !v_cache || !out || (paged && !context_lens)) return ERR_ARG;
    if ((cache_dtype == DT_I8 || cache_dtype == DT_FP8) && (!k_scale || !v_scale)) return ERR_ARG;

    prefill_job j = {q, k_cache, v_cache, qo_dtype, cache_dtype, k_scale, v_scale, block_table, context_lens,
                     batch, seq_len, num_heads, num_kv_heads, head_dim, max_blocks, num_blocks, 0, 0,
                     scale > 0.0f ? (double)scale : 1.0 / sqrt((double)head_dim), out, 0};
    j.cap = (long long)max_blocks * 16;
    if (max_context_len > 0 && j.cap > max_context_len) j.cap = max_context_len;
    for (int b = 0; b < batch; ++b)
    {
        long long L = (paged ? (long long)context_lens[b] : 0) + seq_len;
        if (paged && L > j.cap) L = j.cap;
        if (L > j.max_keys) j.max_keys = L;
    }
    atomic_init(&j.next, 0);

    long long work = (long long)batch * seq_len * (j.max_keys > 0 ? j.max_keys : 1) * num_heads;
    long long items = (long long)batch * num_kv_heads * ((seq_len + PREFILL_TOKENS_PER_ITEM - 1) / PREFILL_TOKENS_PER_ITEM);
    int       threads = work >= (1LL << 20) ? ffo_default_threads() : 1;
    if (threads > items) threads = (int)items;
    if (threads <= 1)
    {
        prefill_worker(&j);
        return 0;
    }
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, prefill_worker, &j);
    for (int i = 0; i < threads; ++i) pthread_join(tids[i], NULL);
    free(tids);
    return 0;
}
