// Shared helpers of the liteinfer_amd HIP sources: error state, element
// types, and the small vector types the MFMA kernels move 16 bytes at a time.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdarg>

#include "../../include/liteinfer_amd.h"

namespace li {

// Records `fmt` as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);
void clear_error();

// Checks the launch that was just enqueued.
int check_launch(const char* what);

// Compute units of the current device, cached per device.
int device_cu_count();

inline int cdiv(int a, int b) { return (a + b - 1) / b; }
inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case LI_F32: return 4;
    case LI_F16: return 2;
    case LI_BF16: return 2;
    case LI_FP8_E4M3: return 1;
    default: return 0;
  }
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace li

// ---------------------------------------------------------------------------
// Device-side types
// ---------------------------------------------------------------------------

typedef __bf16 li_bf16;
typedef _Float16 li_f16;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

// Converts one stored element to fp32.
__device__ __forceinline__ float li_to_float(float x) { return x; }
__device__ __forceinline__ float li_to_float(li_bf16 x) { return (float)x; }
__device__ __forceinline__ float li_to_float(li_f16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T li_from_float(float x);
template <>
__device__ __forceinline__ float li_from_float<float>(float x) { return x; }
template <>
__device__ __forceinline__ li_bf16 li_from_float<li_bf16>(float x) { return (li_bf16)x; }
template <>
__device__ __forceinline__ li_f16 li_from_float<li_f16>(float x) { return (li_f16)x; }

// A quiet NaN of T, from its bit pattern (the sources build with
// -fno-honor-nans, under which a NaN constant is not guaranteed).
template <typename T>
__device__ __forceinline__ T li_quiet_nan() {
  if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, 0x7fc00000u);
  else if constexpr (__is_same(T, li_bf16)) return __builtin_bit_cast(T, (unsigned short)0x7fc0u);
  else return __builtin_bit_cast(T, (unsigned short)0x7e00u);
}

// x clamped to the e4m3 range [-448, 448], a NaN passed through (tested on
// the bits: the sources build with -fno-honor-nans, under which x != x may
// fold to false), so it stores as the e4m3 NaN as torch's cast does.
__device__ __forceinline__ float li_clamp_e4m3(float x) {
  if ((__float_as_uint(x) & 0x7fffffffu) > 0x7f800000u) return x;
  return fminf(fmaxf(x, -448.f), 448.f);
}

// Bit pattern of two 16-bit elements packed low-first, from fp32 values
// rounded to nearest even.
template <typename T>
__device__ __forceinline__ uint32_t li_pack2(float lo, float hi) {
  // A two-element vector conversion, so a single packed convert
  // (v_cvt_pk_bf16_f32 on gfx950) does both roundings.
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  const t2 v = __builtin_convertvector((f2){lo, hi}, t2);
  return __builtin_bit_cast(uint32_t, v);
}

// Wave64 reductions. Every lane gets the result.
__device__ __forceinline__ float li_wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float li_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
