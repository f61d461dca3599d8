// Shared definitions for the gfx950 kernels of libbiops.so: element types and conversions,
// 16-byte vector helpers, error reporting and the per-device property cache.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/biops.h"

namespace biops {

// ------------------------------------------------------------------ element types ----
// bf16 and fp16 travel through memory as raw 16-bit patterns; arithmetic is fp32.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 by the hardware conversion (v_cvt_pk_bf16_f32): round to nearest even; a NaN
// stays a quiet NaN.  Every bf16 result of the library goes through it.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Two values at once (one instruction), element 0 in the low half.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// Typed scalar load/store through fp32.
template <typename T> struct Num;
template <> struct Num<float> {
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ float load(const float* p) { return *p; }
  __device__ static __forceinline__ void store(float* p, float v) { *p = v; }
  __device__ static __forceinline__ float round(float v) { return v; }
  __device__ static __forceinline__ float from_bits(uint32_t b) { return __uint_as_float(b); }
};
template <> struct Num<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float load(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
  __device__ static __forceinline__ void store(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }
  // One conversion: with +0 in the low half, the pair's bits are the rounded value as fp32.
  __device__ static __forceinline__ float round(float v) { return __uint_as_float(f32x2_to_bf16x2_bits(0.f, v)); }
  __device__ static __forceinline__ float from_bits(uint32_t b) { return bf16_bits_to_f32((uint16_t)b); }
  __device__ static __forceinline__ uint16_t to_bits(float v) { return f32_to_bf16_bits(v); }
};
template <> struct Num<f16_t> {
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float load(const f16_t* p) { return f16_bits_to_f32(p->bits); }
  __device__ static __forceinline__ void store(f16_t* p, float v) { p->bits = f32_to_f16_bits(v); }
  __device__ static __forceinline__ float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
  __device__ static __forceinline__ float from_bits(uint32_t b) { return f16_bits_to_f32((uint16_t)b); }
  __device__ static __forceinline__ uint16_t to_bits(float v) { return f32_to_f16_bits(v); }
};

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ host helpers ----
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
int device_cus();  // compute units of the current device (cached)

inline int dtype_bytes(int dt) {
  switch (dt) {
    case BIOPS_F32: return 4;
    case BIOPS_F16: return 2;
    case BIOPS_BF16: return 2;
    case BIOPS_BOOL: return 1;
    default: return 0;
  }
}
inline bool is_float_dtype(int dt) { return dt == BIOPS_F32 || dt == BIOPS_F16 || dt == BIOPS_BF16; }

}  // namespace biops

// Dispatch a block over the three float element types: `T` is bound inside.
#define BIOPS_DISPATCH_FLOAT(dt, ...)                      \
  switch (dt) {                                            \
    case BIOPS_F32: { typedef float T; __VA_ARGS__; break; } \
    case BIOPS_F16: { typedef ::biops::f16_t T; __VA_ARGS__; break; } \
    case BIOPS_BF16: { typedef ::biops::bf16_t T; __VA_ARGS__; break; } \
    default: return ::biops::fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", (int)(dt)); \
  }
