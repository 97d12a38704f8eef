// ffkv_device.h - device-side helpers for the gfx950 paged KV-cache kernels.
//
// Element conversions (round to nearest even, defined NaN and saturation behaviour), vectorised 8-element
// loads/stores of every supported storage type, and the int8 / OCP fp8 e4m3 quantizers.  The conversions are
// integer bit manipulations so that append produces the same bytes on every run and on the CPU checker.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ffkv
{

enum DType : int
{
    F32 = 0,
    F16 = 1,
    BF16 = 2,
    I8 = 3,
    FP8 = 8,
};

__device__ __forceinline__ uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float    u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return u2f(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) & 0x8000u) | 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ uint32_t f32_to_f16(float x)
{
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u;
    if (a < 0x38800000u) return sign | static_cast<uint32_t>(__builtin_rintf(u2f(a) * 16777216.0f));
    a += 0xfffu + ((a >> 13) & 1u);
    a -= 112u << 23;
    return sign | (a >> 13);
}

// OCP e4m3: round half to even, saturate finite values to +-448, NaN -> S.1111.111.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x)
{
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;
    if (a >= 0x43e00000u) return sign | 0x7eu;
    if (a < 0x3c800000u) return sign | static_cast<uint32_t>(__builtin_rintf(u2f(a) * 512.0f));
    a += 0x7ffffu + ((a >> 20) & 1u);
    uint32_t code = (a >> 20) - (120u << 3);
    return sign | (code > 0x7eu ? 0x7eu : code);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t q)
{
    uint32_t mag = q & 0x7fu;
    float    norm = u2f((mag << 20) + (120u << 23));
    float    sub = static_cast<float>(mag) * 0x1p-9f;
    float    v = mag < 8u ? sub : norm;
    v = mag == 0x7fu ? __builtin_nanf("") : v;
    return u2f(f2u(v) | ((q & 0x80u) << 24));
}

// Largest of v (or with SUM its sum) over aligned groups of N lanes (N a power of two up to 32), in every lane of the
// group; for the maximum v is never NaN here (absolute-value maxima that skip NaN).  Every lane must be active.  Quad permutations and the 8- and 16-lane mirrors are DPP
// operands of the compare, the step between 16-lane rows gfx950's row swap: no LDS round trip.
template <int N, bool SUM = false>
__device__ __forceinline__ float group_reduce(float v)
{
    static_assert(N >= 1 && N <= 32 && (N & (N - 1)) == 0, "groups of 1, 2, 4, 8, 16 or 32 lanes");
    auto take = [&v](float o)
    {
        if constexpr (SUM)
            v += o;
        else
            v = o > v ? o : v;
    };
    auto dpp = [](float x, auto ctrl)
    {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                      decltype(ctrl)::value, 0xf, 0xf, false));
    };
    if constexpr (N >= 2) take(dpp(v, std::integral_constant<int, 0xb1>{}));   // quad lanes 1, 0, 3, 2
    if constexpr (N >= 4) take(dpp(v, std::integral_constant<int, 0x4e>{}));   // quad lanes 2, 3, 0, 1
    if constexpr (N >= 8) take(dpp(v, std::integral_constant<int, 0x141>{}));  // lane 7 - i of its 8
    if constexpr (N >= 16) take(dpp(v, std::integral_constant<int, 0x140>{})); // lane 15 - i of its 16
    if constexpr (N >= 32)
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                        false, false);  // rows (0, 0, 2, 2) and (1, 1, 3, 3)
        const float a = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
        const float b = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
        v = SUM ? a + b : (a > b ? a : b);
    }
    return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v)
{
    return group_reduce<N, false>(v);
}

// Sum of v over aligned groups of N lanes, in every lane of the group, with the same lane steps as group_max.
template <int N>
__device__ __forceinline__ float group_sum(float v)
{
    return group_reduce<N, true>(v);
}

__device__ __forceinline__ int32_t quant_i8(float x, float s)
{
    float y = x / s;  // IEEE divide (hipcc keeps fp32 division correctly rounded by default)
    if (y != y) return 0;
    float r = __builtin_rintf(y);
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    return static_cast<int32_t>(r);
}

// The quantizers below give exactly the codes of quant_i8(x, s) and f32_to_e4m3(x / s) without a divide per
// element.  A code depends on the quotient fl(x / s) only through where it falls between the target format's
// rounding boundaries (int8: half-integers; e4m3: the midpoints between neighbouring codes).  y = x * rcp(s) is
// within 1.5 * 2^-23 * |y| of x / s (v_rcp_f32 is accurate to 1 ulp and the product rounds once), at most 3 of
// y's ulps, and fl(x / s) within half an ulp more, so when y lies more than FFKV_QUANT_MARGIN (8) of its ulps from
// every boundary both round to the same code.  Only when it does not (about 2e-5 of random inputs), for e4m3's
// subnormal range and for NaN is the IEEE divide evaluated.  The compiler may fuse the product into the following
// add or subtract; the unrounded product is closer to x / s still, so the bound holds either way.

// 1/s for the quantizers: NaN unless s is positive, normal and finite, which sends every element to the divide.
__device__ __forceinline__ float quant_rcp(float s)
{
    return s >= 0x1p-126f && s < __builtin_huge_valf() ? __builtin_amdgcn_rcpf(s) : __builtin_nanf("");
}

#ifndef FFKV_FP8_HW_CVT
#define FFKV_FP8_HW_CVT 1  // fp8 codes of safe values from v_cvt_pk_fp8_f32 (0: the integer conversion)
#endif

// Distance from a rounding boundary, in ulps of y, beyond which y is "safe" (see above).
#ifndef FFKV_QUANT_MARGIN
#define FFKV_QUANT_MARGIN 8
#endif

// int8: the boundaries are the half-integers: safe when |y - r| < 0.5 - margin * 2^-23 * (|r| + 0.5), r = rint(y).
// Where the test can pass |y| <= |r| + 0.5, so the margin is at least FFKV_QUANT_MARGIN of y's ulps; taking it from
// r leaves y itself only in the difference.  NaN and infinite y fail the test.
__device__ __forceinline__ bool quant_i8_safe(float y, float r)
{
    return __builtin_fabsf(y - r) < __builtin_fmaf(-__builtin_fabsf(r), FFKV_QUANT_MARGIN * 0x1p-23f,
                                                   0.5f - FFKV_QUANT_MARGIN * 0x1p-24f - 0x1p-40f);
}

// e4m3: in the normal range the boundaries are the midpoints between neighbouring codes, where the 20 fp32
// mantissa bits below the 3 kept ones equal 0x80000: safe when they are more than the margin from it and
// |y| >= 2^-6 (one compare, false for NaN).  Smaller y (the subnormal grid, and zero) take the divide; infinite
// and huge y are safe: they clamp to 448, as the conversion saturates them.
__device__ __forceinline__ bool quant_e4m3_safe(float y)
{
    const uint32_t u = f2u(y);
    return __builtin_fabsf(y) >= 0x1p-6f && (u & 0xfffffu) + (FFKV_QUANT_MARGIN - 0x80000u) > 2u * FFKV_QUANT_MARGIN;
}

// Quantize 8 values to packed codes (element i in byte i % 4 of w[i / 4]) with the fast forms; only in a wave
// where some lane has an unsafe value are those values redone with the divide.  int8: s = the row's scale (> 0);
// fp8: s = the head's scale.  fp8 codes of safe values come from the gfx950 conversion v_cvt_pk_fp8_f32 (OCP
// e4m3, round to nearest even) of y clamped to +-448, which equals f32_to_e4m3(y) there: normal-range outputs,
// and y is no tie.
template <bool INT8>
__device__ __forceinline__ void quant8(const float* x, float s, uint32_t* w)
{
    const float rs = quant_rcp(s);
    bool        safe = true;  // fp8: every value of the lane is safe
    uint64_t    bad = 0;      // int8: the lanes holding an unsafe value (one compare and a scalar OR per value)
    if constexpr (INT8)
    {
        // y + 1.5 * 2^23 rounds y to the nearest integer r, ties to even (|y| < 2^22), and holds r in the low bits
        // of the sum: the sum's low byte is r's two's-complement code.  With s = absmax / 127 (the row's finite
        // absmax) |y| <= 127 * (1 + 3 * 2^-24), so r needs no clamp; with any other s, rs is NaN and so is y.
        uint32_t c[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float y = x[i] * rs;
            const float m = y + 0x1.8p23f;
            bad |= __builtin_amdgcn_ballot_w64(!quant_i8_safe(y, m - 0x1.8p23f));
            c[i] = f2u(m);
        }
#pragma unroll
        for (int k = 0; k < 2; ++k)  // bytes 0 of c[4k .. 4k+3]
            w[k] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(c[4 * k + 3], c[4 * k + 2], 0x04000c0cu),
                                         __builtin_amdgcn_perm(c[4 * k + 1], c[4 * k], 0x0c0c0400u), 0x07060100u);
    }
    else
    {
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            y[i] = x[i] * rs;
            safe = safe && quant_e4m3_safe(y[i]);
            y[i] = __builtin_fminf(__builtin_fmaxf(y[i], -448.0f), 448.0f);
        }
#if FFKV_FP8_HW_CVT
#pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * k], y[4 * k + 1], 0, false);
            w[k] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(y[4 * k + 2], y[4 * k + 3], lo, true));
        }
#else
#pragma unroll
        for (int k = 0; k < 2; ++k)
            w[k] = f32_to_e4m3(y[4 * k]) | (f32_to_e4m3(y[4 * k + 1]) << 8) | (f32_to_e4m3(y[4 * k + 2]) << 16) |
                   (f32_to_e4m3(y[4 * k + 3]) << 24);
#endif
    }
    if (__builtin_expect(INT8 ? bad != 0 : !__all(safe), 0))
    {
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float y = x[i] * rs;
            const bool  ok = INT8 ? quant_i8_safe(y, __builtin_rintf(y)) : quant_e4m3_safe(y);
            if (!ok)
            {
                const uint32_t q = INT8 ? static_cast<uint32_t>(quant_i8(x[i], s)) & 0xffu : f32_to_e4m3(x[i] / s);
                const int      sh = 8 * (i & 3);
                w[i / 4] = (w[i / 4] & ~(0xffu << sh)) | (q << sh);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// 8-element vector access.  `p` points at element index `i` (a multiple of 8) of an array of type T.
// ---------------------------------------------------------------------------------------------------------

template <int T>
struct Storage;
template <>
struct Storage<F32>
{
    static constexpr int bytes = 4;
};
template <>
struct Storage<F16>
{
    static constexpr int bytes = 2;
};
template <>
struct Storage<BF16>
{
    static constexpr int bytes = 2;
};
template <>
struct Storage<I8>
{
    static constexpr int bytes = 1;
};
template <>
struct Storage<FP8>
{
    static constexpr int bytes = 1;
};

// Raw 8-element chunk in registers (up to 32 bytes).
struct Raw8
{
    uint32_t w[8];
};

template <int T>
__device__ __forceinline__ void load_raw8(const void* base, size_t i, Raw8& r)
{
    const char* p = static_cast<const char*>(base) + i * Storage<T>::bytes;
    if constexpr (Storage<T>::bytes == 4)
    {
        uint4 a = *reinterpret_cast<const uint4*>(p);
        uint4 b = *reinterpret_cast<const uint4*>(p + 16);
        r.w[0] = a.x, r.w[1] = a.y, r.w[2] = a.z, r.w[3] = a.w;
        r.w[4] = b.x, r.w[5] = b.y, r.w[6] = b.z, r.w[7] = b.w;
    }
    else if constexpr (Storage<T>::bytes == 2)
    {
        uint4 a = *reinterpret_cast<const uint4*>(p);
        r.w[0] = a.x, r.w[1] = a.y, r.w[2] = a.z, r.w[3] = a.w;
    }
    else
    {
        uint2 a = *reinterpret_cast<const uint2*>(p);
        r.w[0] = a.x, r.w[1] = a.y;
    }
}

template <int T>
__device__ __forceinline__ void store_raw8(void* base, size_t i, const Raw8& r)
{
    char* p = static_cast<char*>(base) + i * Storage<T>::bytes;
    if constexpr (Storage<T>::bytes == 4)
    {
        *reinterpret_cast<uint4*>(p) = make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]);
        *reinterpret_cast<uint4*>(p + 16) = make_uint4(r.w[4], r.w[5], r.w[6], r.w[7]);
    }
    else if constexpr (Storage<T>::bytes == 2)
    {
        *reinterpret_cast<uint4*>(p) = make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]);
    }
    else
    {
        *reinterpret_cast<uint2*>(p) = make_uint2(r.w[0], r.w[1]);
    }
}

// Unpack a raw chunk of a float-valued type (F32/F16/BF16) into 8 floats.
template <int T>
__device__ __forceinline__ void unpack8(const Raw8& r, float* x)
{
    if constexpr (T == F32)
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = u2f(r.w[i]);
    }
    else if constexpr (T == BF16)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            x[2 * i] = u2f(r.w[i] << 16);
            x[2 * i + 1] = u2f(r.w[i] & 0xffff0000u);
        }
    }
    else if constexpr (T == F16)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            x[2 * i] = f16_to_f32(r.w[i] & 0xffffu);
            x[2 * i + 1] = f16_to_f32(r.w[i] >> 16);
        }
    }
    else if constexpr (T == I8)
    {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            x[i] = static_cast<float>(static_cast<int8_t>((r.w[i / 4] >> (8 * (i % 4))) & 0xffu));
    }
    else
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = e4m3_to_f32((r.w[i / 4] >> (8 * (i % 4))) & 0xffu);
    }
}

// Pack 8 floats into a raw chunk of a float-valued storage type (rounding to nearest even).
template <int T>
__device__ __forceinline__ void pack8(const float* x, Raw8& r)
{
    if constexpr (T == F32)
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) r.w[i] = f2u(x[i]);
    }
    else if constexpr (T == BF16)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i) r.w[i] = f32_to_bf16(x[2 * i]) | (f32_to_bf16(x[2 * i + 1]) << 16);
    }
    else
    {
        static_assert(T == F16, "pack8: float storage only");
#pragma unroll
        for (int i = 0; i < 4; ++i) r.w[i] = f32_to_f16(x[2 * i]) | (f32_to_f16(x[2 * i + 1]) << 16);
    }
}

// Runtime-typed (F32/F16/BF16) 8-element load/store, for activations whose dtype is a kernel argument.
__device__ __forceinline__ void load_act8(const void* base, int dt, size_t i, float* x)
{
    Raw8 r;
    if (dt == F32)
    {
        load_raw8<F32>(base, i, r);
        unpack8<F32>(r, x);
    }
    else if (dt == F16)
    {
        load_raw8<F16>(base, i, r);
        unpack8<F16>(r, x);
    }
    else
    {
        load_raw8<BF16>(base, i, r);
        unpack8<BF16>(r, x);
    }
}

__device__ __forceinline__ void store_act1(void* base, int dt, size_t i, float x)
{
    if (dt == F32)
        static_cast<float*>(base)[i] = x;
    else if (dt == F16)
        static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(f32_to_f16(x));
    else
        static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(f32_to_bf16(x));
}

// Cross-lane helpers within a wave64.
__device__ __forceinline__ float shfl_xor(float x, int mask) { return __shfl_xor(x, mask, 64); }

}  // namespace ffkv
