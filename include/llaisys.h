/*
 * LLAISYS C ABI -- base types.
 *
 * Binary-compatible with the reference's include/llaisys.h:4-64 (same macros, same enum
 * values, same typedefs) so that a caller built against the reference links and runs
 * against libllaisys.so from llaisys_amd.  The one addition is the device type
 * LLAISYS_DEVICE_AMD = 2 (the reference requires consecutive values, llaisys.h:25), which
 * moves LLAISYS_DEVICE_TYPE_COUNT from 2 to 3.
 */
#ifndef __LLAISYS_H__
#define __LLAISYS_H__

#if defined(_WIN32)
#define __export __declspec(dllexport)
#elif defined(__GNUC__) && ((__GNUC__ >= 4) || (__GNUC__ == 3 && __GNUC_MINOR__ >= 3))
#define __export __attribute__((visibility("default")))
#else
#define __export
#endif

#ifdef __cplusplus
#define __C extern "C"
#include <cstddef>
#include <cstdint>
#else
#define __C
#include <stddef.h>
#include <stdint.h>
#endif

/* Device types (reference llaisys.h:23-28). */
typedef enum {
    LLAISYS_DEVICE_CPU = 0,
    LLAISYS_DEVICE_NVIDIA = 1, /* kept for ABI compatibility; reports 0 devices here */
    LLAISYS_DEVICE_AMD = 2,    /* MI355X / gfx950 through HIP */
    LLAISYS_DEVICE_TYPE_COUNT
} llaisysDeviceType_t;

/* Data types (reference llaisys.h:31-52). */
typedef enum {
    LLAISYS_DTYPE_INVALID = 0,
    LLAISYS_DTYPE_BYTE = 1,
    LLAISYS_DTYPE_BOOL = 2,
    LLAISYS_DTYPE_I8 = 3,
    LLAISYS_DTYPE_I16 = 4,
    LLAISYS_DTYPE_I32 = 5,
    LLAISYS_DTYPE_I64 = 6,
    LLAISYS_DTYPE_U8 = 7,
    LLAISYS_DTYPE_U16 = 8,
    LLAISYS_DTYPE_U32 = 9,
    LLAISYS_DTYPE_U64 = 10,
    LLAISYS_DTYPE_F8 = 11,
    LLAISYS_DTYPE_F16 = 12,
    LLAISYS_DTYPE_F32 = 13,
    LLAISYS_DTYPE_F64 = 14,
    LLAISYS_DTYPE_C16 = 15,
    LLAISYS_DTYPE_C32 = 16,
    LLAISYS_DTYPE_C64 = 17,
    LLAISYS_DTYPE_C128 = 18,
    LLAISYS_DTYPE_BF16 = 19,
} llaisysDataType_t;

/* Opaque stream handle (reference llaisys.h:56); a hipStream_t for the AMD device. */
typedef void *llaisysStream_t;

/* Memory copy directions (reference llaisys.h:59-64). */
typedef enum {
    LLAISYS_MEMCPY_H2H = 0,
    LLAISYS_MEMCPY_H2D = 1,
    LLAISYS_MEMCPY_D2H = 2,
    LLAISYS_MEMCPY_D2D = 3,
} llaisysMemcpyKind_t;

#endif /* __LLAISYS_H__ */
