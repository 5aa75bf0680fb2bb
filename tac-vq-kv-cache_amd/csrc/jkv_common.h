// Shared helpers of the jkv HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "jkv.h"

namespace jkv {

// Thread-local error text; set_error returns the code so call sites can
// `return set_error(JKV_EINVAL, "...")`.
int set_error(int code, const char* fmt, ...);

#define JKV_CHECK_ARG(cond, ...)                          \
  do {                                                    \
    if (!(cond)) return ::jkv::set_error(JKV_EINVAL, __VA_ARGS__); \
  } while (0)

#define JKV_CHECK_HIP(expr)                                              \
  do {                                                                   \
    hipError_t e__ = (expr);                                             \
    if (e__ != hipSuccess)                                               \
      return ::jkv::set_error(JKV_EHIP, "%s failed: %s", #expr,          \
                              hipGetErrorString(e__));                   \
  } while (0)

// Post-launch check (launch configuration errors only; never synchronises).
#define JKV_CHECK_LAUNCH()                                                \
  do {                                                                    \
    hipError_t e__ = hipGetLastError();                                   \
    if (e__ != hipSuccess)                                                \
      return ::jkv::set_error(JKV_EHIP, "kernel launch failed: %s",       \
                              hipGetErrorString(e__));                    \
  } while (0)

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

// Element loads/stores for the three state dtypes.
template <int DT> struct Elem;
template <> struct Elem<JKV_F16> {
  typedef _Float16 T;
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return (float)((const _Float16*)p)[i];
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    ((_Float16*)p)[i] = (_Float16)v;
  }
};
template <> struct Elem<JKV_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    uint32_t b = ((const uint16_t*)p)[i];
    return __uint_as_float(b << 16);
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    // round to nearest even (NaN kept quiet)
    uint32_t u = __float_as_uint(v);
    uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) r = (u >> 16) | 0x40u;
    ((uint16_t*)p)[i] = (uint16_t)r;
  }
};
template <> struct Elem<JKV_F32> {
  typedef float T;
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return ((const float*)p)[i];
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    ((float*)p)[i] = v;
  }
};

// fp16 deploy round trip of an fp32 master value (tables.half().float()).
__device__ __forceinline__ float deploy16(float v) { return (float)(_Float16)v; }

// a - b on eight fp16 lanes as a sign flip of b and four packed adds (IEEE
// a + (-b) is a - b).  Written out because an 8-wide fp16 subtraction is
// otherwise split into scalar subtractions and repacks.
__device__ __forceinline__ half8 sub_h8(half8 a, half8 b) {
  uint4 y = __builtin_bit_cast(uint4, b);
  y.x ^= 0x80008000u;
  y.y ^= 0x80008000u;
  y.z ^= 0x80008000u;
  y.w ^= 0x80008000u;
  return a + __builtin_bit_cast(half8, y);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Map a linear block index so that consecutive logical blocks land on the
// same XCD (hardware dispatches block i to XCD i % 8).  Blocks that share
// input rows then share one L2.  Valid when nblocks is a multiple of 8;
// otherwise the identity is used.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nblocks) {
  if ((nblocks & 7u) != 0u) return bid;
  uint32_t per = nblocks >> 3;
  return (bid & 7u) * per + (bid >> 3);
}

}  // namespace jkv
