// types.h - device and element types of the paged KV-cache library.
//
// Same enumerators, order and helper functions as the reference (include/firefly/types.h:10-95), so code written
// against the reference compiles unchanged.  Two additions: Device::GPU (Device::CUDA is an alias of it, kept for
// source compatibility) and DType::FP8_E4M3 (OCP e4m3 KV caches; the reference has no FP8 type).  The numeric
// values equal the FFKV_DTYPE_* codes of the C ABI (include/ffkv.h).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>

#ifndef FIREFLY_API
#define FIREFLY_API __attribute__((visibility("default")))
#endif

namespace firefly
{

enum class Device : uint8_t
{
    CPU = 0,
    GPU = 1,
    CUDA = GPU,  // the reference's name for the accelerator
};

enum class DType : uint8_t
{
    F32 = 0,
    F16 = 1,
    BF16 = 2,
    I8 = 3,
    I32 = 4,
    I64 = 5,
    U8 = 6,
    UNKNOWN = 7,
    FP8_E4M3 = 8,
};

[[nodiscard]] constexpr std::string_view dtype_to_string(DType dtype) noexcept
{
    switch (dtype)
    {
        case DType::F32:
            return "Float32";
        case DType::F16:
            return "Float16";
        case DType::BF16:
            return "BFloat16";
        case DType::I8:
            return "Int8";
        case DType::I32:
            return "Int32";
        case DType::I64:
            return "Int64";
        case DType::U8:
            return "UInt8";
        case DType::FP8_E4M3:
            return "Float8_e4m3";
        default:
            return "UNKNOWN";
    }
}

// Bytes per element; 0 for UNKNOWN.
[[nodiscard]] constexpr size_t dtype_size(DType dtype)
{
    switch (dtype)
    {
        case DType::F32:
        case DType::I32:
            return 4;
        case DType::F16:
        case DType::BF16:
            return 2;
        case DType::I64:
            return 8;
        case DType::I8:
        case DType::U8:
        case DType::FP8_E4M3:
            return 1;
        default:
            return 0;
    }
}

[[nodiscard]] constexpr size_t element_size(DType dtype) noexcept { return dtype_size(dtype); }

}  // namespace firefly
