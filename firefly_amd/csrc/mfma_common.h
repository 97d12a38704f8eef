// mfma_common.h - matrix-core building blocks shared by the paged decode and prefill kernels (gfx950).
//
// MFMA operand types (bf16 or f16 per cache and q type), exact conversions of 8-bit cache codes, the lane <-> dim
// map of the 16x16x32 operands, the swizzled LDS tile of 16 tokens x D, and wave reductions.
#pragma once

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

// MFMA input element type (bf16 or f16), chosen per cache and q type by kBF below.
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

#ifndef FFKV_I8_BF16
#define FFKV_I8_BF16 0  // int8 caches with bf16 q: bf16 MFMA (1) or f16 MFMA with q split in two (0)
#endif

// bf16 MFMA for bf16 caches, f16 for f16 caches.  Quantized codes are exact in both types (int8 has 8
// significant bits, e4m3 4 bits and exponents -9..8), so they take q's type: then q needs no hi/lo split.
template <int CT, int QT>
constexpr bool kBF = CT == BF16 || (CT == FP8 && QT != F16) || (CT == I8 && QT == BF16 && FFKV_I8_BF16);
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

using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
using f32x2 = float __attribute__((ext_vector_type(2)));

// 4 int8 codes -> 4 bf16 values (two packed words), exact: sign-extending byte converts to f32, then packed
// converts to bf16 (integers of magnitude <= 128 need 8 significant bits).
__device__ __forceinline__ void i8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi)
{
    const float f0 = static_cast<float>(static_cast<int8_t>(w & 0xffu));
    const float f1 = static_cast<float>(static_cast<int8_t>((w >> 8) & 0xffu));
    const float f2 = static_cast<float>(static_cast<int8_t>((w >> 16) & 0xffu));
    const float f3 = static_cast<float>(static_cast<int8_t>(w >> 24));
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{f0, f1}, bf16x2));
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{f2, f3}, bf16x2));
}

// 8 cache codes (one k-step of one lane) as 4 packed 16-bit MFMA words of type bf16 (BF) or f16; exact.  OCP
// e4m3 codes use the gfx950 conversion instructions (scale 1: exact, NaN codes give NaN).
template <int CT, bool BF>
__device__ __forceinline__ u32x4 codes_to_m(uint32_t lo, uint32_t hi)
{
    uint32_t r0, r1, r2, r3;
    if constexpr (CT == I8)
    {
        if constexpr (BF)
        {
            i8x4_to_bf16(lo, r0, r1);
            i8x4_to_bf16(hi, r2, r3);
        }
        else
        {
            i8x4_to_f16(lo, r0, r1);
            i8x4_to_f16(hi, r2, r3);
        }
    }
    else if constexpr (BF)
    {
        r0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
        r1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
        r2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
        r3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
    }
    else
    {
        r0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false));
        r1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true));
        r2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false));
        r3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true));
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

// The same reductions with gfx950's row swaps, which move the values between rows in VALU without an LDS round
// trip: permlane16_swap(x, x) returns rows (0, 0, 2, 2) and (1, 1, 3, 3) of x, permlane32_swap(x, x) halves
// (0, 0) and (1, 1).  Both operand orders give the same bits, and the same bits as xor_max / xor_sum.  (Measured:
// about 4 % faster in the LDS-bound prefill; no gain in the decode, which keeps the LDS permutes.)  swap_max takes
// IEEE maximum (one v_maximum3_f32; fmaxf would first quiet both swapped values, two more instructions), which
// differs from xor_max only for NaN, which it propagates.
__device__ __forceinline__ float swap_max(float x)
{
    const uint32_t u = __float_as_uint(x);
    const auto     r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float    y = __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const uint32_t v = __float_as_uint(y);
    const auto     h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __builtin_elementwise_maximum(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

__device__ __forceinline__ float swap_sum(float x)
{
    const uint32_t u = __float_as_uint(x);
    const auto     r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float    y = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const uint32_t v = __float_as_uint(y);
    const auto     h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

}  // namespace

}  // namespace ffkv
