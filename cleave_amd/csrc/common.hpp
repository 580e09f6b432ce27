// common.hpp -- shared runtime state, error handling and launch helpers for
// libcleave_hip.so.  Every entry point validates its arguments on the host
// before launching anything, so a kernel never sees a shape it was not
// written for.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>

#include "../../include/cleave_hip.h"

namespace ch {

// Library stream (one per process, like the reference's single JIT thread).
hipStream_t stream();
// Opens device 0 and creates the stream on first use; returns status.
int32_t ensure_init();

// Records an error (code + printf-style message).  In abort mode (the
// default, matching cleave-rt's panic) prints to stderr and aborts.
// Returns `code` so callers can `return fail(...)`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Checks a HIP call; on error records it and returns CLEAVE_HIP_ERR_RUNTIME.
int32_t check_hip(hipError_t e, const char* what);

// Buffers of cleave_hip_buf_alloc / cleave_hip_buf_free (a cache of freed
// blocks in runtime.hip).
void* buf_alloc(uint64_t bytes);
void buf_free(void* buf);
// Returns every cached free block to the device; the bytes released.
size_t buf_trim();
size_t buf_cached_bytes();

// Scratch device memory owned by the library (grown on demand, never shrunk).
// `slot` (0 .. kScratchSlots-1) selects an independent buffer.
constexpr int kScratchSlots = 16;
void* scratch(int slot, size_t bytes);
// Same buffer, but a failed allocation returns nullptr without recording an
// error (for callers that have another way to do the work).
void* scratch_try(int slot, size_t bytes);

// Number of compute units (for grid sizing of persistent/strided kernels).
int num_cus();

// a * b * c for non-negative factors, or -1 when the product exceeds int64
// (so that no operand length matches it).
inline int64_t count3(int64_t a, int64_t b, int64_t c) {
    if (a == 0 || b == 0 || c == 0) return 0;
    if (a > INT64_MAX / b) return -1;
    const int64_t ab = a * b;
    return ab > INT64_MAX / c ? -1 : ab * c;
}

// Workspace of the allocation-free entry point (cleave_hip_reduce_sum_f32_noalloc):
// a static device array of kNoAllocFloats floats, its device address resolved
// once at init with the library's device current.  nullptr when that failed.
// Every call shares it: calls that overlap on one device race.
constexpr int kNoAllocFloats = 16384;  // 64 KiB
float* noalloc_workspace();

// Tensor operands of the device entry points must be device memory: a host
// address handed to a kernel faults the GPU.  Fails with CLEAVE_HIP_ERR_ARG
// when `p` is not device (or managed) memory of this process, or when its
// allocation ends fewer than `bytes` bytes after `p`.  The `_host` entry
// points take host arrays instead.
int32_t require_device(const char* fn, const char* what, const void* p, uint64_t bytes);

}  // namespace ch

#define CH_INIT_OR_RETURN()                       \
    do {                                          \
        int32_t _st = ch::ensure_init();          \
        if (_st != CLEAVE_HIP_OK) return _st;     \
    } while (0)

#define CH_HIP(expr)                                                   \
    do {                                                               \
        int32_t _st = ch::check_hip((expr), #expr);                    \
        if (_st != CLEAVE_HIP_OK) return _st;                          \
    } while (0)

#define CH_LAUNCHED(name)                                               \
    do {                                                                \
        int32_t _st = ch::check_hip(hipGetLastError(), name);           \
        if (_st != CLEAVE_HIP_OK) return _st;                           \
    } while (0)

// Device-operand check: `CH_DEVICE(fn, ptr, bytes)` returns on failure.
#define CH_DEVICE(fn, p, bytes)                                                       \
    do {                                                                              \
        int32_t _st = ch::require_device((fn), #p, (const void*)(p), (uint64_t)(bytes)); \
        if (_st != CLEAVE_HIP_OK) return _st;                                         \
    } while (0)

// Argument checks used by every entry point.
#define CH_REQUIRE(cond, ...)                                     \
    do {                                                          \
        if (!(cond)) return ch::fail(CLEAVE_HIP_ERR_ARG, __VA_ARGS__); \
    } while (0)
