// Error types, HIP checks and small shared definitions for the native library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace cllm {

// Typed errors; the C ABI maps each type to its error code (reference
// src/common/cuda_check.h:10-20, src/capi/cudallm_capi.cpp:24-30).  Device errors are a type of
// their own instead of being recognised by a substring of the message.
struct ArgError : std::runtime_error { using std::runtime_error::runtime_error; };
struct FormatError : std::runtime_error { using std::runtime_error::runtime_error; };
struct IoError : std::runtime_error { using std::runtime_error::runtime_error; };
struct DeviceError : std::runtime_error { using std::runtime_error::runtime_error; };
struct StateError : std::runtime_error { using std::runtime_error::runtime_error; };
// A step on a full sequence.  The reference raises a plain runtime_error here
// (src/engine/engine.cpp:118 via CUDALLM_CHECK), which its C ABI reports as CUDALLM_ERR_INTERNAL
// (src/capi/cudallm_capi.cpp:22-29); this type keeps that code.
struct SequenceFull : std::runtime_error { using std::runtime_error::runtime_error; };

[[noreturn]] void throw_hip(hipError_t err, const char* expr, const char* file, int line);

// File-level weight type codes and tensor dtype codes of the .cudallm format.
enum class WType : int { BF16 = 1, INT8 = 3, INT4 = 4 };
enum class TDType : uint32_t { F32 = 0, BF16 = 1, F16 = 2, I8 = 3, I4X2 = 4 };
enum class Epilogue : int { STORE = 0, ADD = 1, SWIGLU = 2 };

const char* wtype_name(WType w);

}  // namespace cllm

#define CLLM_HIP(expr)                                                      \
    do {                                                                    \
        hipError_t cllm_e_ = (expr);                                        \
        if (cllm_e_ != hipSuccess) ::cllm::throw_hip(cllm_e_, #expr, __FILE__, __LINE__); \
    } while (0)

#define CLLM_REQUIRE(cond, msg)                       \
    do {                                              \
        if (!(cond)) throw ::cllm::ArgError(msg);     \
    } while (0)

#define CLLM_INTERNAL(cond, msg)                      \
    do {                                              \
        if (!(cond)) throw std::logic_error(msg);     \
    } while (0)
