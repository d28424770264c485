// int4 codebook decode helpers shared by the weight-decode kernels and the fused small-M W4A8 GEMM.
//   level(c, s) = clamp(rint_half_even(f32(codebook[c]) * f32(s)), -127, 127), a NaN product -> 0
//   (reference h3turbo/h3/qlinear.py:157-204)
// A scale's 16 levels form a byte table in 4 registers: byte c of word w = level(codebook[4w + c], s).
#pragma once
#include "h3k_common.hpp"

namespace h3k {

template <int SD>
__device__ __forceinline__ float load_scale(const void* s, int64_t idx) {
  if (SD == H3K_FP8E4M3) return fp8e4m3fn_to_f32(static_cast<const uint8_t*>(s)[idx]);
  if (SD == H3K_F16) return f16_to_f32(static_cast<const uint16_t*>(s)[idx]);
  if (SD == H3K_BF16) return bf16_to_f32(static_cast<const uint16_t*>(s)[idx]);
  return static_cast<const float*>(s)[idx];
}

__device__ __forceinline__ uint32_t level(float cbv, float s) {
  float p = cbv * s;
  if (p != p) p = 0.0f;
  p = __builtin_amdgcn_fmed3f(__builtin_rintf(p), -127.0f, 127.0f);
  return static_cast<uint32_t>(static_cast<int>(p)) & 0xFFu;
}

__device__ __forceinline__ uint32_t lut_lookup(const uint32_t (&lut)[4], uint32_t sel, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(lut[1], lut[0], sel);  // sel: nibble & 7 per byte
  const uint32_t hi = __builtin_amdgcn_perm(lut[3], lut[2], sel);
  return __builtin_amdgcn_perm(hi, lo, 0x03020100u | b3);  // b3: 4 in bytes whose nibble has bit 3 set
}


// The 16-entry byte table of scale s (cbv = the codebook in registers).
__device__ __forceinline__ void build_lut(const float (&cbv)[16], float s, uint32_t (&lut)[4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w)
    lut[w] = level(cbv[4 * w], s) | (level(cbv[4 * w + 1], s) << 8) | (level(cbv[4 * w + 2], s) << 16) |
             (level(cbv[4 * w + 3], s) << 24);
}

// build_lut without the per-level NaN test where none can occur: a finite scale times a finite codebook entry is
// finite (the clamp takes +-inf products of the general path to +-127 anyway).  Same table as build_lut.
__device__ __forceinline__ void build_lut_fast(const float (&cbv)[16], bool cb_finite, float s, uint32_t (&lut)[4]) {
  if (cb_finite && __builtin_isfinite(s)) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t v = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float p = __builtin_amdgcn_fmed3f(__builtin_rintf(cbv[4 * w + c] * s), -127.0f, 127.0f);
        v |= (static_cast<uint32_t>(static_cast<int>(p)) & 0xFFu) << (8 * c);
      }
      lut[w] = v;
    }
  } else {
    build_lut(cbv, s, lut);
  }
}

__device__ __forceinline__ bool all_finite(const float (&cbv)[16]) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 16; ++i) ok = ok && __builtin_isfinite(cbv[i]);
  return ok;
}

// 4 packed bytes (k = 2j: low nibble, 2j + 1: high nibble) -> 8 levels in k order, as two words.
__device__ __forceinline__ void lut_decode_word(const uint32_t (&lut)[4], uint32_t pk, uint32_t& lo4, uint32_t& hi4) {
  const uint32_t dlo = lut_lookup(lut, pk & 0x07070707u, (pk >> 1) & 0x04040404u);
  const uint32_t dhi = lut_lookup(lut, (pk >> 4) & 0x07070707u, (pk >> 5) & 0x04040404u);
  lo4 = __builtin_amdgcn_perm(dhi, dlo, 0x05010400u);  // k 0..3 of the word
  hi4 = __builtin_amdgcn_perm(dhi, dlo, 0x07030602u);  // k 4..7
}

}  // namespace h3k
