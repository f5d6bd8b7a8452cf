// Shared host/device helpers of the gfx950 SageAttention library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sageattn_mi355x.h"

namespace sage {

// ---------------------------------------------------------------- host side
// Records a formatted message for sage_last_error() on this thread; returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's message (called on entry of every public function).
void clear_error();
// Maps a pending launch error to SAGE_ERR_HIP.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- device side
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef int int16_t_ __attribute__((ext_vector_type(16)));
typedef float float16_t_ __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Two packed 16-bit values (one dword) -> two floats; exact for fp16 and bf16.
template <bool BF16>
__device__ __forceinline__ float2_t unpack2(uint32_t w) {
  if constexpr (BF16) {
    float2_t r;
    r.x = __uint_as_float(w << 16);
    r.y = __uint_as_float(w & 0xffff0000u);
    return r;
  } else {
    return __builtin_convertvector(__builtin_bit_cast(half2_t, w), float2_t);
  }
}

// Two floats -> one dword of two fp16 (round to nearest even).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  float2_t t = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(t, half2_t));
}

// Two floats -> one dword of two bf16 (round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  float2_t t = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(t, bf16x2_t));
}

// ---------------------------------------------------------------- INT8 quantisation (bit-exact)
// csrc/attn_gfx11.cu:192 of the reference: absmax floor of a scale group.
constexpr float kAmaxFloor = 1e-7f;

// float_to_int8 of csrc/attn_gfx11.cu:85-92: u = fp32 t + (t >= 0 ? 0.5 : -0.5),
// clamp to [-128, 127], truncate toward zero (NaN -> 0).  Computed here as
// trunc(t + copysign(0.5, t)) with v_cvt_i32_f32 (saturating, NaN -> 0) and an
// integer clamp, which gives the same value for every input: the two forms
// differ in u only for t = -0 (u = -0.5 instead of 0.5, both truncate to 0),
// and clamping after truncation equals truncating after clamping because the
// bounds are integers.  The add must not fuse with the caller's multiply,
// hence contraction off.
__device__ __forceinline__ int round_half_away_i8(float t) {
#pragma clang fp contract(off)
  const float u = t + __builtin_copysignf(0.5f, t);
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(u));  // saturating, NaN -> 0 (the ISA rule)
  return min(max(r, -128), 127);
}

__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
         ((static_cast<uint32_t>(c) & 0xffu) << 16) | ((static_cast<uint32_t>(d) & 0xffu) << 24);
}

}  // namespace sage
