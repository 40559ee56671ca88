// Shared device/host helpers for the gfx950 attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/alpx.h"

namespace alpx {

typedef _Float16 f16_t;
typedef __bf16 bf16_t;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// log2(e): scores are kept in the base-2 domain so the softmax uses the
// hardware exp2 (v_exp_f32) directly.
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(bf16_t x) { return static_cast<float>(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return static_cast<f16_t>(x); }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return static_cast<bf16_t>(x); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Stable two-branch logistic function: never overflows for finite x.
__device__ __forceinline__ float stable_sigmoid(float x) {
  if (x >= 0.0f) {
    float z = __expf(-x);
    return 1.0f / (1.0f + z);
  }
  float z = __expf(x);
  return z / (1.0f + z);
}

// Logistic function as 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and
// reciprocal (about 2 ulp): saturates to exactly 0 and 1 without overflow
// trouble (2^(+large) = inf gives 1 / inf = 0), so it needs no branch.
__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-x * kLog2e));
}

// Vector of 8 16-bit elements of type T, the MFMA k=32 operand of one lane.
template <typename T> struct Vec8;
template <> struct Vec8<f16_t> { typedef f16x8 type; };
template <> struct Vec8<bf16_t> { typedef bf16x8 type; };

template <typename T> struct Vec4;
template <> struct Vec4<f16_t> { typedef f16x4 type; };
template <> struct Vec4<bf16_t> { typedef bf16x4 type; };
template <> struct Vec4<float> { typedef f32x4 type; };

// 16x16x4 fp32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16].
__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Within each group of
// 16 lanes, lane i = 4k + q supplies the address of 4 consecutive 16-bit
// elements (row R_k, columns C + 4q .. C + 4q + 3 of a row-major tile);
// lane j of the group receives column C + j of rows R_0 .. R_3.  Used to
// read a row-major [row][col] LDS tile as MFMA operands that need 4
// consecutive rows of one column per lane.
__device__ __forceinline__ f16x4 lds_read_tr4(const f16_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}
__device__ __forceinline__ bf16x4 lds_read_tr4(const bf16_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// Raw buffer resource over `bytes` bytes at `base` (loads past the end read
// zero instead of touching memory).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Blocks of `kernel` (with `block` threads, `lds` dynamic bytes) that fit on
// one CU at once, times the CU count of the current device (cached per
// kernel and device).
int resident_blocks(const void* kernel, int block, size_t lds);
// CU count of the current device (cached per device).
int multiprocessor_count();

inline size_t dtype_size(int dtype) {
  return dtype == ALPX_F32 ? 4 : 2;
}

inline bool dtype_ok(int dtype) {
  return dtype == ALPX_F32 || dtype == ALPX_F16 || dtype == ALPX_BF16;
}

// Host-side error slot shared by every entry point (abi.hip).
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

// Current value of kernel-choice override `which` (enum alpx_override):
// the environment as read at load, or the last alpx_set_override.
int override_value(int which);

}  // namespace alpx
