// Shared device helpers and host-side error plumbing of the h3k library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <type_traits>
#include <utility>

#include "h3k.h"

namespace h3k {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Compile-time loop: f(std::integral_constant<int, i>{}) for i in [0, N).  Register arrays indexed through it
// only ever see constant indices, so they are promoted to registers before any unrolling happens.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ------------------------------------------------------------------------------------------ host errors
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Checks the launch that just happened; returns H3K_OK or H3K_ELAUNCH with the message recorded.
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline bool is_pow4(int r) { return r == 4 || r == 16 || r == 64 || r == 256 || r == 1024; }

// ------------------------------------------------------------------------------------------ number formats
// Materialise an fp32 value: stops the backend from fusing the operation that produced it with a later
// narrowing conversion (e.g. fptrunc(fmul) -> v_fma_mixlo_f16 rounds once, where the reference rounds to fp32
// first and then to f16: the two differ when the fp32 result is an exact f16 tie).
__device__ __forceinline__ float fp32_round_point(float f) {
  __asm__ volatile("" : "+v"(f));
  return f;
}

// bf16 bits -> float (exact)
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// float -> bf16 bits, round to nearest even (NaN kept quiet).  hipcc lowers the __bf16 conversion to the
// gfx950 hardware RNE conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b));
}

// float -> value of bf16, as float
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_bits(f)); }

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);  // IEEE RNE
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}
__device__ __forceinline__ float round_f16(float f) { return f16_to_f32(f32_to_f16_bits(f)); }

// OCP E4M3FN byte -> float: bias 7, subnormals m * 2^-9, S.1111.111 is NaN, no infinities.
__device__ __forceinline__ float fp8e4m3fn_to_f32(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24, e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 0) {
    v = static_cast<float>(m) * 0.001953125f;  // m / 8 * 2^-6, exact
  } else if (e == 15 && m == 7) {
    v = __uint_as_float(0x7FC00000u);
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(v) | s);
}

// Wave-local LDS ordering: every lane's earlier LDS accesses complete before any later one is issued.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// max that propagates NaN (IEEE 754-2019 maximum: v_maximum_f32 / v_maximum3_f32 on gfx950), like torch's amax
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float wave_nan_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace h3k
