// Shared helpers for the gfx950 kernels: status reporting, element types,
// vector types for MFMA operands and the XCD-aware work-group remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/vgo.h"

namespace vgo {

// ---------------------------------------------------------------- status ----
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

#define VGO_REQUIRE(cond, msg)                      \
  do {                                              \
    if (!(cond)) return ::vgo::fail(VGO_EINVAL, msg); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// ------------------------------------------------------------ vector types --
typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;

// Round-to-nearest-even conversions (the hardware v_cvt_pk_bf16_f32 rounds RNE).
__device__ __forceinline__ float to_f32(bf16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(float x) { return x; }
template <typename T>
__device__ __forceinline__ T from_f32(float x) { return static_cast<T>(x); }

// ------------------------------------------------------- XCD-aware remap ----
// MI355X dispatches consecutive work-group ids round-robin over its 8 XCDs,
// each with a private L2.  This bijection on [0, total) hands every XCD one
// contiguous range of logical tasks, so tasks that share operands (same
// attention head, neighbouring rows) land in the same L2.
constexpr int kNumXcd = 8;
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  if (total < kNumXcd) return pid;
  const int per = (total + kNumXcd - 1) / kNumXcd;
  int tall = total % kNumXcd;
  if (tall == 0) tall = kNumXcd;
  const int xcd = pid % kNumXcd;
  const int local = pid / kNumXcd;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

}  // namespace vgo
