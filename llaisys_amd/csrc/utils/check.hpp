// Error reporting for the LLAISYS C ABI.
//
// Same convention as the reference (src/utils/check.hpp:7-88): a failed check prints an
// "[ERROR] ..." line with the location to stderr and throws a std::runtime_error or
// std::invalid_argument.  The C entry points do not catch, so through ctypes a failure
// ends the process, exactly as with the reference library.
#pragma once

#include <iostream>
#include <stdexcept>
#include <string>

#define LLAISYS_WHERE " from " << __func__ << " at " << __FILE__ << ":" << __LINE__ << "."

#define LLAISYS_FAIL(EXC, PRINTED, THROWN)                                \
    do {                                                                  \
        std::cerr << "[ERROR] " << PRINTED << LLAISYS_WHERE << std::endl; \
        throw EXC(THROWN);                                                \
    } while (0)

#define EXCEPTION_UNSUPPORTED_DEVICE \
    LLAISYS_FAIL(std::runtime_error, "Unsupported device", "Unsupported device")

#define EXCEPTION_UNSUPPORTED_DATATYPE(DT__)                                                  \
    LLAISYS_FAIL(std::runtime_error,                                                          \
                 "Unsupported data type: " << llaisys::utils::dtype_to_str(DT__),             \
                 "Unsupported data type")

#define TO_BE_IMPLEMENTED() \
    LLAISYS_FAIL(std::runtime_error, "Unimplemented function", "Unimplemented function")

#define CHECK_ARGUMENT(COND, MSG)                                                    \
    do {                                                                             \
        if (!(COND)) LLAISYS_FAIL(std::invalid_argument, "Invalid argument: " << MSG, MSG); \
    } while (0)

#define ASSERT(COND, MSG)                                                               \
    do {                                                                                \
        if (!(COND)) {                                                                  \
            std::cerr << "[ERROR] " << MSG << std::endl                                 \
                      << "Assertion failed: " << #COND << LLAISYS_WHERE << std::endl;   \
            throw std::runtime_error("Assertion failed");                               \
        }                                                                               \
    } while (0)

#define EXCEPTION_SHAPE_MISMATCH \
    LLAISYS_FAIL(std::invalid_argument, "Shapes mismatch", "Shapes mismatch")
#define EXCEPTION_DATATYPE_MISMATCH \
    LLAISYS_FAIL(std::invalid_argument, "Datatypes mismatch", "Datatypes mismatch")

// Every further argument must equal the first (shapes or dtypes).
#define CHECK_SAME(ON_FAIL, FIRST, ...)               \
    do {                                              \
        for (const auto &other__ : {__VA_ARGS__}) {   \
            if (!((FIRST) == other__)) { ON_FAIL; }   \
        }                                             \
    } while (0)
#define CHECK_SAME_SHAPE(FIRST, ...) CHECK_SAME(EXCEPTION_SHAPE_MISMATCH, FIRST, __VA_ARGS__)
#define CHECK_SAME_DTYPE(FIRST, ...) CHECK_SAME(EXCEPTION_DATATYPE_MISMATCH, FIRST, __VA_ARGS__)

// Every tensor must live on the device (type and id) of the first.
#define CHECK_SAME_DEVICE(FIRST, ...)                                                       \
    do {                                                                                    \
        for (const auto &t__ : {__VA_ARGS__}) {                                             \
            if ((FIRST)->deviceType() != t__->deviceType()                                  \
                || (FIRST)->deviceId() != t__->deviceId()) {                                \
                std::cerr << "[ERROR] Input tensors must be on the same device!" << std::endl \
                          << "Device mismatch" << LLAISYS_WHERE << std::endl;               \
                throw std::runtime_error("device mismatch");                                \
            }                                                                               \
        }                                                                                   \
    } while (0)
