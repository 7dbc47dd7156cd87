// Data-type helpers shared by the host code.
#pragma once

#include "llaisys.h"

#include <cstring>
#include <stdexcept>

namespace llaisys::utils {

// Bytes per element (reference src/utils/types.hpp:18-62).
inline size_t dsize(llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_BYTE:
    case LLAISYS_DTYPE_BOOL:
    case LLAISYS_DTYPE_I8:
    case LLAISYS_DTYPE_U8:
    case LLAISYS_DTYPE_F8: return 1;
    case LLAISYS_DTYPE_I16:
    case LLAISYS_DTYPE_U16:
    case LLAISYS_DTYPE_F16:
    case LLAISYS_DTYPE_BF16:
    case LLAISYS_DTYPE_C16: return 2;
    case LLAISYS_DTYPE_I32:
    case LLAISYS_DTYPE_U32:
    case LLAISYS_DTYPE_F32:
    case LLAISYS_DTYPE_C32: return 4;
    case LLAISYS_DTYPE_I64:
    case LLAISYS_DTYPE_U64:
    case LLAISYS_DTYPE_F64:
    case LLAISYS_DTYPE_C64: return 8;
    case LLAISYS_DTYPE_C128: return 16;
    default: throw std::invalid_argument("Unsupported or invalid data type.");
    }
}

// Names as printed by the reference (src/utils/types.hpp:64-108).
inline const char *dtype_to_str(llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_BYTE: return "byte";
    case LLAISYS_DTYPE_BOOL: return "bool";
    case LLAISYS_DTYPE_I8: return "int8";
    case LLAISYS_DTYPE_I16: return "int16";
    case LLAISYS_DTYPE_I32: return "int32";
    case LLAISYS_DTYPE_I64: return "int64";
    case LLAISYS_DTYPE_U8: return "uint8";
    case LLAISYS_DTYPE_U16: return "uint16";
    case LLAISYS_DTYPE_U32: return "uint32";
    case LLAISYS_DTYPE_U64: return "uint64";
    case LLAISYS_DTYPE_F8: return "float8";
    case LLAISYS_DTYPE_F16: return "float16";
    case LLAISYS_DTYPE_BF16: return "bfloat16";
    case LLAISYS_DTYPE_F32: return "float32";
    case LLAISYS_DTYPE_F64: return "float64";
    case LLAISYS_DTYPE_C16: return "complex16";
    case LLAISYS_DTYPE_C32: return "complex32";
    case LLAISYS_DTYPE_C64: return "complex64";
    case LLAISYS_DTYPE_C128: return "complex128";
    default: throw std::invalid_argument("Unsupported or invalid data type.");
    }
}

// Host-side widening of the 16-bit float formats, used only for printing (tensorDebug).
inline float bf16_bits_to_f32(uint16_t b) {
    uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float f16_bits_to_f32(uint16_t h);

} // namespace llaisys::utils
