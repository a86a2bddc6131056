// Internal helpers shared by the translation units of libmi355x_bench.so.
//
// Conventions of the C-ABI (declared in include/mi355x_bench.h):
//   * every entry point returns MB_OK (0) or a negative MB_ERR_* code and never
//     throws, aborts or exits across the boundary;
//   * the message of the most recent failure on the calling thread is kept in a
//     thread-local buffer returned by mb_last_error();
//   * device memory is owned by the caller; launches are asynchronous on the
//     caller's stream and no entry point synchronises the device.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/mi355x_bench.h"

namespace mb {

// Set the thread-local error message; returns `code` so call sites can write
// `return fail(MB_ERR_INVALID, "...")`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Translate a HIP status into the ABI convention, recording where it happened.
int hip_status(hipError_t status, const char* what);

// Check the status of the most recent asynchronous launch on this thread.
inline int launch_status(const char* kernel) {
  return hip_status(hipGetLastError(), kernel);
}

inline bool aligned(const void* ptr, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) == 0;
}

inline bool power_of_two(uint64_t value) { return value && !(value & (value - 1)); }

// Registry of kernels, so the host can query hipFuncGetAttributes by name
// (register count, LDS and scratch bytes) for the resource audit.
struct KernelEntry {
  const char* name;
  const void* func;
};
void register_kernel(const char* name, const void* func);

// MB_OK for a matrix format with kernels; MB_ERR_UNSUPPORTED for TF32.
int matrix_format_check(int format, const char* entry);

struct KernelRegistrar {
  KernelRegistrar(const char* name, const void* func) { register_kernel(name, func); }
};

}  // namespace mb

#define MB_CONCAT_IMPL(a, b) a##b
#define MB_CONCAT(a, b) MB_CONCAT_IMPL(a, b)
// Register a kernel (or a template instantiation) under a stable name.
#define MB_REGISTER_KERNEL(name, func) \
  static mb::KernelRegistrar MB_CONCAT(mb_registrar_, __COUNTER__)(name, reinterpret_cast<const void*>(func))
