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

// Device address of the current device's static scratch (VGO_ATTN_STATIC_SCRATCH_BYTES,
// csrc/scratch.hip), looked up once per device.
int static_scratch(void** out);

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

// max(||row||_2, eps) of a row held as lane l's elements 4(l + 64i) + j in
// v[i][j] (chunks past `chunks` ignored): squares summed with fused
// multiply-adds over i, then j, then a butterfly over the wave, so every lane
// gets the same value.  normalize_rows and the fused LayerNorm row pass both
// use this order, so their unit rows agree bit for bit.
template <int kChunks>
__device__ __forceinline__ float row_l2_denominator(const float (&v)[kChunks][4], int lane,
                                                    int chunks, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kChunks; ++i)
    if (i * 64 + lane < chunks) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = fmaf(v[i][j], v[i][j], ss);
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  return fmaxf(sqrtf(ss), eps);
}

constexpr int kNormChunks = 8;  // normalize_rows: dim <= 4 * 64 * 8

// Four consecutive elements as one vector load / store (4-element aligned).
template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  using type = f32x4;
};
template <>
struct Vec4<bf16_t> {
  using type = bf16x4;
};
template <>
struct Vec4<f16_t> {
  using type = f16x4;
};

// A restore weight as the value type sees it: `w.to(value.dtype)` in the
// reference's projection (token_merging.py:408-413); fp32 values keep it.
template <typename T>
__device__ __forceinline__ float weight_as_value(float w) {
  return to_f32(from_f32<T>(w));
}
template <>
__device__ __forceinline__ float weight_as_value<float>(float w) {
  return w;
}

// Product rounded to the value type (bf16/f16 multiply semantics), fp32 as is.
template <typename T>
__device__ __forceinline__ float rounded_product(float y, float w) {
  return to_f32(from_f32<T>(y * w));
}
template <>
__device__ __forceinline__ float rounded_product<float>(float y, float w) {
  return y * w;
}

template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
  const typename Vec4<T>::type v = *reinterpret_cast<const typename Vec4<T>::type*>(p);
  return f32x4{to_f32(v[0]), to_f32(v[1]), to_f32(v[2]), to_f32(v[3])};
}

template <typename T>
__device__ __forceinline__ void store4(T* p, f32x4 v) {
  typename Vec4<T>::type o;
  o[0] = from_f32<T>(v[0]);
  o[1] = from_f32<T>(v[1]);
  o[2] = from_f32<T>(v[2]);
  o[3] = from_f32<T>(v[3]);
  *reinterpret_cast<typename Vec4<T>::type*>(p) = o;
}


// Value held by lane (lane ^ kXor), kXor = 1 or 2, within each group of four
// lanes: a DPP quad permutation, which stays in the VALU (a ds_bpermute
// shuffle goes through the LDS unit and waits for it).  The four lanes of a
// group must be active together.
template <int kXor>
__device__ __forceinline__ float quad_xor(float v) {
  static_assert(kXor == 1 || kXor == 2, "quad_xor: lane ^ 1 or lane ^ 2");
  constexpr int kCtrl = kXor == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

// LayerNorm over the 64 channels of one head held by four consecutive lanes
// (16 each, channel d0 + j in v[j]); statistics in fp32, two passes.  w and b
// point at the affine parameters of this lane's 16 channels.
__device__ __forceinline__ void head_layer_norm(float* v, const float* w, const float* b,
                                                float eps) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += v[j];
  s += quad_xor<1>(s);
  s += quad_xor<2>(s);
  const float mean = s / 64.0f;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    v[j] = v[j] - mean;  // kept centred for the scaling below
    q = fmaf(v[j], v[j], q);
  }
  q += quad_xor<1>(q);
  q += quad_xor<2>(q);
  // v_rsq_f32 (about 1 ulp; var + eps >= eps > 0 is a normal number), as the
  // reference's GPU LayerNorm takes rsqrt rather than a rounded 1 / sqrt.
  const float rstd = __builtin_amdgcn_rsqf(q / 64.0f + eps);
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = fmaf(v[j] * rstd, w[j], b[j]);
}

// ------------------------------------------------------------ LDS DMA ----
// global_load_lds_dword{,x4}: lane i of the wave writes 4 (16) bytes at LDS
// byte address M0 + 4i (16i).  Issued from inline asm so the compiler does not
// track these loads (its tracking would wait for all of them before any LDS
// read); kernels wait for them with wait_vmem.  Because vmcnt is in order, any
// wait the compiler inserts for its own memory operations (a spill reload)
// also waits for every DMA in flight, so loops that issue DMAs must not spill.
// No kernel of this library otherwise uses M0.  An SALU write of M0 needs one
// wait state before an LDS-DMA instruction reads it (the s_nop).
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  typedef const __attribute__((address_space(3))) char* lds_ptr;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)(p)));
}
// Global address = base (wave-uniform, SGPRs) + 32-bit byte offset (per lane).
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t offset, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(offset), "s"(base) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* base, uint32_t offset, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :: "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(offset), "s"(base) : "memory");
}
// Per-lane 64-bit global address.
__device__ __forceinline__ void lds_dma16_addr(const void* addr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(addr) : "memory");
}
// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace vgo
