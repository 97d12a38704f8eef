// ffkv_device.h - device-side helpers for the gfx950 paged KV-cache kernels.
//
// Element conversions (round to nearest even, defined NaN and saturation behaviour), vectorised 8-element
// loads/stores of every supported storage type, and the int8 / OCP fp8 e4m3 quantizers.  The conversions are
// integer bit manipulations so that append produces the same bytes on every run and on the CPU checker.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

__device__ __forceinline__ int32_t quant_i8(float x, float s)
{
    float y = x / s;  // IEEE divide (hipcc keeps fp32 division correctly rounded by default)
    if (y != y) return 0;
    float r = __builtin_rintf(y);
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    return static_cast<int32_t>(r);
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
