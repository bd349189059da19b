// Shared helpers of the gfx950 kernels: bf16 storage conversions, wavefront reductions, the status /
// error-message plumbing of the C ABI and launch wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

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

// Eight consecutive row elements as loaded (bf16: one 16-byte load; fp32: two), unpacked to fp32 on use, so a
// kernel can issue every row's loads before it reads the first one.
template <typename T>
struct Raw8;
template <>
struct Raw8<bf16_t> {
  u32x4 v;
  __device__ __forceinline__ void load(const bf16_t *p) { v = *reinterpret_cast<const u32x4 *>(p); }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ float get(int k) const { return (k & 1) ? hi_bf(v[k >> 1]) : lo_bf(v[k >> 1]); }
};
template <>
struct Raw8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float *p) {
    a = *reinterpret_cast<const f32x4 *>(p);
    b = *reinterpret_cast<const f32x4 *>(p + 4);
  }
  __device__ __forceinline__ void zero() { a = b = f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ float get(int k) const { return k < 4 ? a[k] : b[k - 4]; }
};

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

// max of three / two floats as one v_max3_f32 / v_max_f32. Written as asm: the compiler's fmaxf quiets
// signalling NaNs with an extra max per operand; the attention kernels' scores are MFMA outputs or -inf, never NaN.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ float vmax2(float a, float b) {
  float d;
  asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
// max over lanes l, l ^ 16, l ^ 32, l ^ 48 with gfx950's lane swaps (VALU, no LDS round trip):
// v_permlane32_swap(x, x) returns {x of lanes l % 32, x of lanes l % 32 + 32} and v_permlane16_swap(x, x)
// {x of the even 16-lane row of l's pair, x of the odd one}
__device__ __forceinline__ float max_lane_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float m = vmax2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return vmax2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// The 16 x 16 x 32 MFMA operand "column c0 + lane % 16 of a row-major bf16 LDS tile (PITCH elements per row) at
// rows r0 + 4 g .. + 3 and r0 + 16 + 4 g .. + 3" (g = lane / 16) as one bf16x8 -- a transposed fragment -- from
// two gfx950 transpose reads ds_read_b64_tr_b16: within each 16-lane group, source lane s reads 4 consecutive
// columns c0 + 4 (s % 4) .. + 3 of row R0 + s / 4, and output lane j receives column c0 + j at rows R0 .. R0 + 3.
// PITCH % 4 == 0 and c0 % 4 == 0 keep every read 8-byte aligned.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
template <int PITCH>
__device__ __forceinline__ bf16x8 lds_tr_frag(const bf16_t *tile, int r0, int c0, int lane) {
  static_assert(PITCH % 4 == 0, "8-byte aligned transpose reads");
  const int g = lane >> 4, s = lane & 15;
  const bf16_t *p0 = tile + (r0 + 4 * g + (s >> 2)) * PITCH + c0 + 4 * (s & 3);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4_t *)(const __attribute__((address_space(3))) bf16_t *)p0);
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4_t *)(const __attribute__((address_space(3))) bf16_t *)(p0 + 16 * PITCH));
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
  return __builtin_bit_cast(bf16x8, s16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
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

// Raise a kernel's dynamic-LDS limit once per process, thread-safe: each call site keeps its own once_flag
// and status (the hipFuncSetAttribute status of the first call, seen by every later caller).
#define VK_RAISE_LDS_ONCE(kernel, bytes, what)                                                                 \
  do {                                                                                                        \
    static std::once_flag vk_lds_once_;                                                                       \
    static hipError_t vk_lds_status_ = hipSuccess;                                                            \
    std::call_once(vk_lds_once_, [] {                                                                         \
      vk_lds_status_ = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),                           \
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)); \
    });                                                                                                       \
    if (vk_lds_status_ != hipSuccess)                                                                         \
      return ::vk::fail(VK_ERR_LAUNCH, "%s: cannot reserve %zu bytes of LDS", what, static_cast<size_t>(bytes)); \
  } while (0)

static inline bool vk_aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
