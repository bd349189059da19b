// Shared helpers of the gfx950 kernels: bf16 storage conversions, wavefront reductions, the status /
// error-message plumbing of the C ABI and launch wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/viktor_hip.h"

namespace vk {

typedef uint16_t bf16_t;  // raw bf16 storage
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// CUs of the current device, queried once per process (256 on MI355X; the launch heuristics use it).
inline int device_cus_cached() {
  static int cus = -1;
  if (cus < 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32: round to nearest even (the rounding torch and Triton
// use), NaN -> quiet NaN; one instruction per pair of values.
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f)); }

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Low / high bf16 of a packed 32-bit word.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
  const f32x2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

// Butterfly reductions over the 64 lanes of a wavefront (every lane gets the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Reduction over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

}  // namespace vk

// ---- host side: status + message -------------------------------------------------------------
namespace vk {
int fail(int code, const char *fmt, ...);
int launch_status(const char *what);
}  // namespace vk

#define VK_CHECK_ARG(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::vk::fail(VK_ERR_ARG, __VA_ARGS__);     \
  } while (0)

#define VK_STREAM(s) reinterpret_cast<hipStream_t>(s)

static inline bool vk_aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
