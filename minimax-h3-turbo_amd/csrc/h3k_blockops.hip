// Token-wise ops of the DiT block around the W4A8 linears, fused: RMSNorm + AdaLN modulation in one pass.
//
// Reference h3turbo/h3/model.py:64-65 (_rms: F.rms_norm with the weight in x.dtype) and :106-109 (_scale_shift_:
// h.mul_(1 + scale).add_(shift), in place in the activation dtype).  Per token row t (bf16, length k):
//   r    = 1 / sqrt(sum_e fp32(x[e])^2 / k + eps)                   fp32; the sum's order is this kernel's own
//   n[e] = bf16(fp32(x[e]) * r * w[e])                              F.rms_norm on bf16: fp32 math, one rounding
//   h[e] = bf16(bf16(n[e] * bf16(1 + scale[m][e])) + shift[m][e])   m = the token's modulation row
// One workgroup per R rows (R = 4 for many rows, else 1), k / 8 threads of 8 elements: each thread issues its
// loads of the R rows' values and of the weight words at once, and reuses the weight, shift and scale words (L2)
// for all R rows, reloading shift and scale only where the modulation row changes.  The squares are summed per
// thread, then across each wavefront by an xor tree, then over the wavefronts in order through LDS.  x is read once
// and h written once.  One wavefront per row (the row in registers, the weight words reloaded per row) ran at
// 0.34-0.41 of HBM.
#include "h3k_common.hpp"

namespace h3k {

// 8 consecutive values of a weight, shift, scale or gate vector as bf16 bits, two per word: bf16 vectors as they
// are, fp32 ones rounded to bf16 here (round-to-nearest-even, as torch's .to(torch.bfloat16), which the reference
// applies to them before use), so the caller needs no conversion pass.
template <bool VF32>
__device__ __forceinline__ u32x4 load8_bf16(const void* __restrict__ base, int64_t idx) {
  if constexpr (VF32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    const float4 a = p[0], b = p[1];
    return u32x4{f32_to_bf16_bits(a.x) | (f32_to_bf16_bits(a.y) << 16), f32_to_bf16_bits(a.z) | (f32_to_bf16_bits(a.w) << 16),
                 f32_to_bf16_bits(b.x) | (f32_to_bf16_bits(b.y) << 16), f32_to_bf16_bits(b.z) | (f32_to_bf16_bits(b.w) << 16)};
  } else {
    return *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + idx);
  }
}

// GATED: the row is first x + y * gate (the gated residual add below, same rounding), stored back into x, and that
// row is normalised and modulated: the block's residual add followed by the next RMSNorm + modulation, x read once.
template <int R, bool GATED, bool VF32>
__global__ __launch_bounds__(1024) void rms_modulate_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                            int k, const void* __restrict__ w,
                                                            const void* __restrict__ shift,
                                                            const void* __restrict__ scale, int64_t ldm,
                                                            const int32_t* __restrict__ row_of_token, float eps,
                                                            uint16_t* __restrict__ h, int64_t ldh,
                                                            const uint16_t* __restrict__ y, int64_t ldy,
                                                            const void* __restrict__ gate, int64_t ldg) {
  __shared__ float s_part[R][16];
  const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
  const int nw = static_cast<int>(blockDim.x) >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * R;
  const int nr = static_cast<int>(min(static_cast<int64_t>(R), rows - t0));
  const int e0 = tid * 8;
  const bool on = e0 < k;
  const u32x4 zero{0, 0, 0, 0};
  // every load of the thread goes out at once: its 8 values of each of the R rows, then the weight words
  u32x4 v[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    v[r] = on && r < nr ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (t0 + r) * ldx + e0)) : zero;
  if constexpr (GATED) {
    u32x4 yv[R], gv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool live = on && r < nr;
      const int64_t mg = live && row_of_token ? row_of_token[t0 + r] : 0;
      yv[r] = live ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(y + (t0 + r) * ldy + e0)) : zero;
      gv[r] = live ? load8_bf16<VF32>(gate, mg * ldg + e0) : zero;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t word = 0;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int sft = 16 * half;
          const float xe = bf16_to_f32((v[r][j] >> sft) & 0xFFFFu), ye = bf16_to_f32((yv[r][j] >> sft) & 0xFFFFu);
          const float ge = bf16_to_f32((gv[r][j] >> sft) & 0xFFFFu);
          word |= f32_to_bf16_bits(fp32_round_point(xe + fp32_round_point(ye * ge))) << sft;
        }
        o[j] = word;
      }
      v[r] = o;
      if (on && r < nr)
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(const_cast<uint16_t*>(x) + (t0 + r) * ldx + e0));
    }
  }
  const u32x4 wv = on ? load8_bf16<VF32>(w, e0) : zero;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = __uint_as_float(v[r][j] << 16), b = __uint_as_float(v[r][j] & 0xFFFF0000u);
      ss = ss + fp32_round_point(a * a);
      ss = ss + fp32_round_point(b * b);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
    if (lane == 0) s_part[r][wave] = ss;
  }
  __syncthreads();
  if (!on) return;
  int64_t mprev = -1;
  u32x4 shv = zero, scv = zero;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nr) break;
    const int64_t t = t0 + r;
    const int64_t m = row_of_token ? row_of_token[t] : 0;
    if (m != mprev) {  // the modulation row's words, reloaded only when it changes
      shv = load8_bf16<VF32>(shift, m * ldm + e0);
      scv = load8_bf16<VF32>(scale, m * ldm + e0);
      mprev = m;
    }
    float tot = s_part[r][0];
    for (int i = 1; i < nw; ++i) tot = tot + s_part[r][i];  // the same fixed order in every thread
    const float rr = 1.0f / sqrtf(fp32_round_point(fp32_round_point(tot / static_cast<float>(k)) + eps));
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int sft = 16 * half;
        const float xe = bf16_to_f32((v[r][j] >> sft) & 0xFFFFu);
        const float we = bf16_to_f32((wv[j] >> sft) & 0xFFFFu);
        const float n = round_bf16(fp32_round_point(fp32_round_point(xe * rr) * we));
        const float one_plus = round_bf16(bf16_to_f32((scv[j] >> sft) & 0xFFFFu) + 1.0f);
        const float h1 = round_bf16(fp32_round_point(n * one_plus));
        const float h2 = fp32_round_point(h1 + bf16_to_f32((shv[j] >> sft) & 0xFFFFu));
        word |= f32_to_bf16_bits(h2) << sft;
      }
      o[j] = word;
    }
    *reinterpret_cast<u32x4*>(h + t * ldh + e0) = o;
  }
}

// Gated residual add (reference h3turbo/h3/model.py:112-115, _gate_: x[tokens].addcmul_(y[tokens], gate[row].to(
// x.dtype)), in place, bf16):
//   x[t][e] = bf16(fp32(x[t][e]) + fp32(y[t][e]) * fp32(g[m][e]))    m = the token's modulation row
// g is the gate already rounded to bf16.  The product of two bf16 values is exact in fp32, so this is one fp32
// rounding of the sum (with or without an fma), then the rounding to bf16: torch's addcmul on bf16 tensors.
// One thread per 8 elements (16-byte loads and stores); x and y are read once, x written once.
template <bool VF32>
__global__ __launch_bounds__(256) void gated_add_kernel(uint16_t* __restrict__ x, int64_t ldx,
                                                        const uint16_t* __restrict__ y, int64_t ldy,
                                                        const void* __restrict__ gate, int64_t ldg,
                                                        const int32_t* __restrict__ row_of_token, int64_t rows,
                                                        int chunks) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= rows * chunks) return;
  const int64_t t = u / chunks;
  const int e0 = static_cast<int>(u - t * chunks) * 8;
  const int64_t m = row_of_token[t];
  u32x4* xp = reinterpret_cast<u32x4*>(x + t * ldx + e0);
  const u32x4 xv = __builtin_nontemporal_load(xp);
  const u32x4 yv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(y + t * ldy + e0));
  const u32x4 gv = load8_bf16<VF32>(gate, m * ldg + e0);
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t word = 0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int sft = 16 * half;
      const float xe = bf16_to_f32((xv[j] >> sft) & 0xFFFFu), ye = bf16_to_f32((yv[j] >> sft) & 0xFFFFu);
      const float ge = bf16_to_f32((gv[j] >> sft) & 0xFFFFu);
      word |= f32_to_bf16_bits(fp32_round_point(xe + fp32_round_point(ye * ge))) << sft;
    }
    o[j] = word;
  }
  __builtin_nontemporal_store(o, xp);
}

}  // namespace h3k

using namespace h3k;

extern "C" int h3k_gated_add(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, int64_t ldg,
                             const int32_t* row_of_token, int64_t rows, int64_t k, int gate_dtype, void* stream) {
  if (gate_dtype != H3K_BF16 && gate_dtype != H3K_F32)
    return fail(H3K_EINVAL, "gate dtype code %d: bf16 or f32", gate_dtype);
  if (rows < 0 || k <= 0 || k % 8 || k > (int64_t(1) << 24))
    return fail(H3K_EINVAL, "k=%lld must be a positive multiple of 8", (long long)k);
  if (ldx < k || ldy < k || ldg < k) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (rows == 0) return H3K_OK;
  if (!x || !y || !gate || !row_of_token) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(x, 16) || !aligned(y, 16) || !aligned(gate, 16) || ldx % 8 || ldy % 8 || ldg % 8)
    return fail(H3K_EINVAL, "rows must be 16-byte aligned (strides multiples of 8 elements)");
  const int chunks = static_cast<int>(k / 8);
  const int64_t threads = rows * chunks;
  if ((threads + 255) / 256 > 0x7FFFFFFF) return fail(H3K_EINVAL, "too many elements for one launch");
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (gate_dtype == H3K_F32)
    hipLaunchKernelGGL(gated_add_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(x), ldx, static_cast<const uint16_t*>(y), ldy, gate, ldg, row_of_token,
                       rows, chunks);
  else
    hipLaunchKernelGGL(gated_add_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(x), ldx, static_cast<const uint16_t*>(y), ldy, gate, ldg, row_of_token,
                       rows, chunks);
  return check_launch("gated_add");
}

template <bool GATED>
static void launch_rms_modulate(const void* x, int64_t ldx, int64_t rows, int64_t k, const void* w, const void* shift,
                                const void* scale, int64_t ldm, const int32_t* row_of_token, float eps, void* h,
                                int64_t ldh, const void* y, int64_t ldy, const void* gate, int64_t ldg, bool vf32,
                                void* stream) {
  const unsigned threads = static_cast<unsigned>((k / 8 + 63) / 64 * 64);  // k <= 8192: at most 1024
  // 4 rows per workgroup share the weight words once there are rows enough to fill the CUs (12602 x 5120: 60-65 us
  // against 75-79 us with one row, 87-90 with 8); one row per workgroup below (777 x 3072: 4.9 against 7.1 us)
  const bool four = rows >= 2048;
  const dim3 grid(static_cast<unsigned>(four ? (rows + 3) / 4 : rows));
#define H3K_RM(R, F)                                                                                                 \
  hipLaunchKernelGGL((rms_modulate_kernel<R, GATED, F>), grid, dim3(threads), 0, static_cast<hipStream_t>(stream),  \
                     static_cast<const uint16_t*>(x), ldx, rows, static_cast<int>(k), w, shift, scale, ldm,          \
                     row_of_token, eps, static_cast<uint16_t*>(h), ldh, static_cast<const uint16_t*>(y), ldy, gate,  \
                     ldg)
  if (four) {
    if (vf32) H3K_RM(4, true);
    else H3K_RM(4, false);
  } else {
    if (vf32) H3K_RM(1, true);
    else H3K_RM(1, false);
  }
#undef H3K_RM
}

extern "C" int h3k_rms_modulate(const void* x, int64_t ldx, int64_t rows, int64_t k, const void* w, const void* shift,
                                const void* scale, int64_t ldm, const int32_t* row_of_token, float eps, void* h,
                                int64_t ldh, int vec_dtype, void* stream) {
  if (vec_dtype != H3K_BF16 && vec_dtype != H3K_F32)
    return fail(H3K_EINVAL, "weight/shift/scale dtype code %d: bf16 or f32", vec_dtype);
  if (rows < 0 || k <= 0 || k % 8 || k > 16 * 512)
    return fail(H3K_EINVAL, "k=%lld must be a positive multiple of 8 up to 8192", (long long)k);
  if (ldx < k || ldh < k || ldm < k) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (rows == 0) return H3K_OK;
  if (!x || !w || !shift || !scale || !h) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(shift, 16) || !aligned(scale, 16) || !aligned(h, 16) || ldx % 8 ||
      ldh % 8 || ldm % 8)
    return fail(H3K_EINVAL, "rows and vectors must be 16-byte aligned (strides multiples of 8 elements)");
  if (rows > 0x7FFFFFFF) return fail(H3K_EINVAL, "too many rows for one launch");
  launch_rms_modulate<false>(x, ldx, rows, k, w, shift, scale, ldm, row_of_token, eps, h, ldh, nullptr, 0, nullptr, 0,
                             vec_dtype == H3K_F32, stream);
  return check_launch("rms_modulate");
}

extern "C" int h3k_gated_add_rms_modulate(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate,
                                          int64_t ldg, int64_t rows, int64_t k, const void* w, const void* shift,
                                          const void* scale, int64_t ldm, const int32_t* row_of_token, float eps,
                                          void* h, int64_t ldh, int vec_dtype, void* stream) {
  if (vec_dtype != H3K_BF16 && vec_dtype != H3K_F32)
    return fail(H3K_EINVAL, "gate/weight/shift/scale dtype code %d: bf16 or f32", vec_dtype);
  if (rows < 0 || k <= 0 || k % 8 || k > 16 * 512)
    return fail(H3K_EINVAL, "k=%lld must be a positive multiple of 8 up to 8192", (long long)k);
  if (ldx < k || ldy < k || ldg < k || ldh < k || ldm < k) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (rows == 0) return H3K_OK;
  if (!x || !y || !gate || !w || !shift || !scale || !h || !row_of_token) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(x, 16) || !aligned(y, 16) || !aligned(gate, 16) || !aligned(w, 16) || !aligned(shift, 16) ||
      !aligned(scale, 16) || !aligned(h, 16) || ldx % 8 || ldy % 8 || ldg % 8 || ldh % 8 || ldm % 8)
    return fail(H3K_EINVAL, "rows and vectors must be 16-byte aligned (strides multiples of 8 elements)");
  if (rows > 0x7FFFFFFF) return fail(H3K_EINVAL, "too many rows for one launch");
  launch_rms_modulate<true>(x, ldx, rows, k, w, shift, scale, ldm, row_of_token, eps, h, ldh, y, ldy, gate, ldg,
                            vec_dtype == H3K_F32, stream);
  return check_launch("gated_add_rms_modulate");
}
