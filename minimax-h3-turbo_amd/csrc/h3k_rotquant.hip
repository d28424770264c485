// Block-Hadamard (ConvRot) rotation + per-token int8 quantisation for gfx950.
//
// Numerics (reference h3turbo/h3/qlinear.py:105-115, 267-292, quant_mode "ck"/"eager"):
//   y32[j] = fp32( sum_i x[i] * H[i, j] )       H = kron(H4, ..., H4) / sqrt(rot), exact dyadic entries
//   amax   = max_j |y32[j]|   ("ck")   or   max_j |round_dtype(y32[j])|   ("eager")
//   xs     = max(amax / 127, 1e-30)                                   (fp32, returned)
//   s      = round_dtype(xs), 0 -> finfo(dtype).tiny
//   q[j]   = clamp(rint_half_even(round_dtype(round_dtype(y32[j]) / s)), -128, 127)
// The rotation is a fast Walsh-Hadamard transform in float64: the products are exact (entries +-2^-p) and
// every partial sum of <= 1024 bf16 / f16 terms is exact in fp64 unless a block spans more than ~2^37 in
// magnitude, so the single rounding to fp32 reproduces the reference's fp64 matmul bit for bit.
//
// Rotation sizes that are not powers of 4 (8, 32, 128, 512: an extension the reference rejects) use
//   H = kron(H2, H4, ..., H4) / sqrt(rot),  H2 = [[1, 1], [1, -1]] as the most significant factor,
// computed as the exact fp64 sum of +-x times fp64(1/sqrt(rot)) = RN(sqrt 2) * 2^-(log2(rot) + 1) / 2, then
// rounded to fp32: one fp64 rounding (1/sqrt(rot) is irrational) and the rounding to fp32.
//
// Fast path (rot = 256 or 128, bf16/f16): one wavefront per row, 4 rows per 256-thread workgroup.  A 256-block spans
// 16 lanes x 16 elements; the four base-4 digits of the in-block index are brought into registers two at a
// time by two LDS transposes (bf16 input, then fp64 mid-values), so every butterfly is register-local.  The
// whole row stays in registers as rounded 16-bit values until its absmax is known; x is read once and q
// written once.
#include <mutex>

#include "h3k_common.hpp"

namespace h3k {

typedef __attribute__((address_space(3))) const uint16_t* lds_u16p;

// h[r][31:16] = the 16-bit LDS value at src + 32 r bytes, h[r][15:0] kept, r = 0..15; the loads and their wait are
// one statement, so no use of h can be scheduled before the data has arrived.
__device__ __forceinline__ void load16_d16_hi(uint32_t (&h)[16], lds_u16p src) {
  __asm__ volatile(
      "ds_read_u16_d16_hi %0, %16\n\tds_read_u16_d16_hi %1, %16 offset:32\n\t"
      "ds_read_u16_d16_hi %2, %16 offset:64\n\tds_read_u16_d16_hi %3, %16 offset:96\n\t"
      "ds_read_u16_d16_hi %4, %16 offset:128\n\tds_read_u16_d16_hi %5, %16 offset:160\n\t"
      "ds_read_u16_d16_hi %6, %16 offset:192\n\tds_read_u16_d16_hi %7, %16 offset:224\n\t"
      "ds_read_u16_d16_hi %8, %16 offset:256\n\tds_read_u16_d16_hi %9, %16 offset:288\n\t"
      "ds_read_u16_d16_hi %10, %16 offset:320\n\tds_read_u16_d16_hi %11, %16 offset:352\n\t"
      "ds_read_u16_d16_hi %12, %16 offset:384\n\tds_read_u16_d16_hi %13, %16 offset:416\n\t"
      "ds_read_u16_d16_hi %14, %16 offset:448\n\tds_read_u16_d16_hi %15, %16 offset:480\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "+v"(h[0]), "+v"(h[1]), "+v"(h[2]), "+v"(h[3]), "+v"(h[4]), "+v"(h[5]), "+v"(h[6]), "+v"(h[7]), "+v"(h[8]),
        "+v"(h[9]), "+v"(h[10]), "+v"(h[11]), "+v"(h[12]), "+v"(h[13]), "+v"(h[14]), "+v"(h[15])
      : "v"(src)
      : "memory");
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// y = x @ H4 on four values (H4 symmetric): (s - 2d, s - 2c, s - 2b, s - 2a) with s = a + b + c + d.
__device__ __forceinline__ void h4(double& a, double& b, double& c, double& d) {
  const double s = (a + b) + (c + d);
  const double na = fma(d, -2.0, s), nb = fma(c, -2.0, s), nc = fma(b, -2.0, s), nd = fma(a, -2.0, s);
  a = na;
  b = nb;
  c = nc;
  d = nd;
}

// y = x @ H2 on two values.
__device__ __forceinline__ void h2(double& a, double& b) {
  const double s = a + b, d = a - b;
  a = s;
  b = d;
}

constexpr double kSqrt2 = 0x1.6a09e667f3bcdp+0;  // RN(sqrt(2))

// 1/sqrt(2^log2) in fp64: exact for even log2, RN(sqrt 2) * 2^-(log2 + 1) / 2 for odd log2.
__device__ __forceinline__ double rot_scale(int log2) {
  return (log2 & 1) ? kSqrt2 * ldexp(1.0, -(log2 + 1) / 2) : ldexp(1.0, -log2 / 2);
}

template <bool F16>
__device__ __forceinline__ float to_f32_16(uint32_t bits) {
  return F16 ? f16_to_f32(bits) : bf16_to_f32(bits);
}
template <bool F16>
__device__ __forceinline__ uint32_t round_bits_16(float f) {
  return F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
}

// Activations applied to the input as it is loaded (ACT 1: [gate | up] rows, silu(gate) * up; ACT 2: tanh GELU),
// each op rounded to the activation dtype like the torch ops they replace: F.silu(gate).mul_(up) (reference
// h3turbo/h3/qlinear.py:376-379) and F.gelu(x, approximate="tanh"), both with fp32 math.
constexpr int kActNone = 0, kActSwiglu = 1, kActGeluTanh = 2;

template <bool F16>
__device__ __forceinline__ float round16(float f) {
  return F16 ? round_f16(f) : round_bf16(f);
}

template <bool F16>
__device__ __forceinline__ uint32_t swiglu_word(uint32_t g2, uint32_t u2) {
  uint32_t r = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float g = to_f32_16<F16>((g2 >> (16 * h)) & 0xFFFFu), u = to_f32_16<F16>((u2 >> (16 * h)) & 0xFFFFu);
    const float d = fp32_round_point(1.0f + expf(-g));
    const float sl = round16<F16>(fp32_round_point(g / d));
    r |= round_bits_16<F16>(fp32_round_point(sl * u)) << (16 * h);
  }
  return r;
}

template <bool F16>
__device__ __forceinline__ uint32_t gelu_tanh_word(uint32_t x2) {
  constexpr float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  constexpr float kKappa = 0.044715f;
  uint32_t r = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float x = to_f32_16<F16>((x2 >> (16 * h)) & 0xFFFFu);
    const float cube = fp32_round_point(fp32_round_point(x * x) * x);
    const float inner = fp32_round_point(kBeta * fp32_round_point(x + fp32_round_point(kKappa * cube)));
    const float y = fp32_round_point(fp32_round_point(0.5f * x) * fp32_round_point(1.0f + tanhf(inner)));
    r |= round_bits_16<F16>(y) << (16 * h);
  }
  return r;
}

// GELU-tanh of every 16-bit input, one table per activation dtype (0 bf16, 1 f16), filled once per device by
// gelu_lut_kernel, which runs gelu_tanh_word itself on each input: the table is that function, value for value.
// The activation-fused quantiser then reads two table entries per word instead of evaluating tanhf twice.
__device__ uint16_t g_gelu_lut[2][65536];

template <bool F16>
__global__ __launch_bounds__(256) void gelu_lut_kernel() {
  const uint32_t v = blockIdx.x * 256u + threadIdx.x;  // grid 256 x 256: every 16-bit input once
  g_gelu_lut[F16][v] = static_cast<uint16_t>(gelu_tanh_word<F16>(v) & 0xFFFFu);
}

__device__ __forceinline__ uint32_t gelu_lut_word(const uint16_t* __restrict__ lut, uint32_t x2) {
  return static_cast<uint32_t>(lut[x2 & 0xFFFFu]) | (static_cast<uint32_t>(lut[x2 >> 16]) << 16);
}

// LDS geometry of the fast path (per wave, per 16-lane group g)
constexpr int kInStride = 16 * 16 + 16;  // uint16 per group: 16 rows of 16 + pad (skews groups by 8 banks)
constexpr int kMidRow = 17;              // doubles per mid-transpose row (odd: conflict-free 64-bit access)
constexpr int kMidStride = 16 * kMidRow + 4;

// WPR wavefronts share a row (1 or 4): wave w of the row owns the 256-blocks (p * WPR + w) * 4 + g, so long rows
// keep NPASS (and the registers holding the row) small; the row's absmax is then combined through LDS.
// Row layout: element e of row r is at x[r * ldx + (e >> hshift) * hstride + (e & (2^hshift - 1))]; hshift = 31
// is a plain row, hshift = log2(head_dim) reads a head-major [heads, rows, head_dim] tensor as rows of
// heads * head_dim (head_dim >= 16, so a lane's 16 consecutive elements stay inside one head).
// ROT 256, or 128: the 256 elements of a lane group are then two 128-blocks (bit 7 of the index separates them),
// with H2 on bit 6 in place of H4 on bits 6-7, and the scale applied at the end.
template <int NPASS, int WPR, bool F16, bool EAGER, int ACT = kActNone, int ROT = 256>
__global__ __launch_bounds__(256) void rotquant256_kernel(const uint16_t* __restrict__ x, int64_t rows, int k,
                                                          int64_t ldx, int hshift, int64_t hstride,
                                                          int8_t* __restrict__ q, int64_t ldq, float* __restrict__ xs,
                                                          const uint16_t* __restrict__ lut) {
  static_assert(WPR == 1 || WPR == 4, "one row per wavefront or one row per workgroup");
  // The 16-bit input transpose and the fp64 mid transpose of a pass never overlap in time, so they share one
  // buffer: 35 KiB per workgroup instead of 44 KiB lets four workgroups (4 waves per SIMD) share a CU.
  static_assert(kInStride * 2 <= kMidStride * 8, "input transpose must fit the mid-transpose area");
  __shared__ __attribute__((aligned(16))) double s_mid[4][4 * kMidStride];
  __shared__ float s_amax[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (4 / WPR) + wave / WPR;
  const int wr = wave % WPR;
  if (row >= rows) return;  // WPR == 4: the whole workgroup leaves together
  const int g = lane >> 4, l = lane & 15;
  const int nb = k >> 8;
  const uint16_t* xr = x + row * ldx;

  u32x4 raw[NPASS][2];
#pragma unroll
  for (int p = 0; p < NPASS; ++p) {
    const int b = (p * WPR + wr) * 4 + g;
    if (b < nb) {
      const int e = b * 256 + l * 16;
      const u32x4* src = reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(e >> hshift) * hstride +
                                                        (e & ((1 << hshift) - 1)));
      raw[p][0] = __builtin_nontemporal_load(src);
      raw[p][1] = __builtin_nontemporal_load(src + 1);
      if (ACT == kActSwiglu) {  // plain rows of 2k: gate at e, up at k + e
        const u32x4* up = reinterpret_cast<const u32x4*>(xr + k + e);
        const u32x4 u0 = __builtin_nontemporal_load(up), u1 = __builtin_nontemporal_load(up + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          raw[p][0][i] = swiglu_word<F16>(raw[p][0][i], u0[i]);
          raw[p][1][i] = swiglu_word<F16>(raw[p][1][i], u1[i]);
        }
      } else if (ACT == kActGeluTanh) {
        if (lut) {  // the table of gelu_tanh_word (wave-uniform choice)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            raw[p][0][i] = gelu_lut_word(lut, raw[p][0][i]);
            raw[p][1][i] = gelu_lut_word(lut, raw[p][1][i]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            raw[p][0][i] = gelu_tanh_word<F16>(raw[p][0][i]);
            raw[p][1][i] = gelu_tanh_word<F16>(raw[p][1][i]);
          }
        }
      }
    } else {
      raw[p][0] = u32x4{0, 0, 0, 0};
      raw[p][1] = u32x4{0, 0, 0, 0};
    }
  }

  uint16_t* tin = reinterpret_cast<uint16_t*>(&s_mid[wave][g * kMidStride]);
  double* tmid = &s_mid[wave][g * kMidStride];
  uint32_t yb[NPASS][8];  // rounded rotation, two 16-bit values per word, contiguous elements l*16 ..
  uint32_t hv[16] = {};   // bf16 input words (value in the high half, zero low half)
  float amax = 0.0f;

#pragma unroll
  for (int p = 0; p < NPASS; ++p) {
    // (blocks past the row hold zeros: their rotation is 0 and leaves the absmax alone)
    // (1) transpose the 16-bit input: lane l then holds elements l + 16*r, r = 0..15 (digits 2,3 local)
    wave_lds_sync();
    *reinterpret_cast<u32x4*>(tin + l * 16) = raw[p][0];
    *reinterpret_cast<u32x4*>(tin + l * 16 + 8) = raw[p][1];
    wave_lds_sync();
    // The 1/16 of H256 (or of 1/sqrt(128) = sqrt(2)/16) is applied here, to the fp32 inputs: a power-of-two
    // scaling, exact for every bf16 and f16 value (the smallest, 2^-133 and 2^-24, stay fp32-representable), so
    // every partial sum below is the exact sum of the scaled terms and the transforms need no scale step.
    double v[16];
    if constexpr (!F16) {
      // bf16 -> fp32 is the bf16 bits in the high half of a word whose low half is zero: ds_read_u16_d16_hi loads
      // them there and keeps the low half, which these registers only ever hold as zero (no shift per element).
      const lds_u16p src = (lds_u16p)(tin + l);
      load16_d16_hi(hv, src);
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = static_cast<double>(__uint_as_float(hv[r]) * 0.0625f);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = static_cast<double>(to_f32_16<F16>(tin[r * 16 + l]) * 0.0625f);
    }
    // (2) digit 2 (r = d2 + 4*d3) and digit 3
#pragma unroll
    for (int d3 = 0; d3 < 4; ++d3) h4(v[4 * d3], v[4 * d3 + 1], v[4 * d3 + 2], v[4 * d3 + 3]);
    if constexpr (ROT == 256) {
#pragma unroll
      for (int d2 = 0; d2 < 4; ++d2) h4(v[d2], v[d2 + 4], v[d2 + 8], v[d2 + 12]);
    } else {  // H2 on bit 6 of each 128-block
#pragma unroll
      for (int d2 = 0; d2 < 4; ++d2) {
        h2(v[d2], v[d2 + 4]);
        h2(v[d2 + 8], v[d2 + 12]);
      }
    }
    // (3) transpose the fp64 mid-values back: lane l then holds elements 16*l + j, j = 0..15 (digits 0,1 local)
    wave_lds_sync();  // the input reads above are done before the area is overwritten
#pragma unroll
    for (int r = 0; r < 16; ++r) tmid[r * kMidRow + l] = v[r];
    wave_lds_sync();
    double w[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = tmid[l * kMidRow + j];
    // (4) digit 0 (j = d0 + 4*d1), then digit 1
#pragma unroll
    for (int d1 = 0; d1 < 4; ++d1) h4(w[4 * d1], w[4 * d1 + 1], w[4 * d1 + 2], w[4 * d1 + 3]);
#pragma unroll
    for (int d0 = 0; d0 < 4; ++d0) h4(w[d0], w[d0 + 4], w[d0 + 8], w[d0 + 12]);
    if constexpr (ROT == 128) {  // exact sums of the scaled terms, then the one fp64 rounding of the sqrt(2) factor
#pragma unroll
      for (int j = 0; j < 16; ++j) w[j] *= kSqrt2;
    }
    // (5) one rounding to fp32, absmax, one rounding to the activation dtype
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      const float y0 = static_cast<float>(w[j]), y1 = static_cast<float>(w[j + 1]);
      uint32_t pair;
      if constexpr (F16) {
        pair = round_bits_16<F16>(y0) | (round_bits_16<F16>(y1) << 16);
      } else {  // one RNE conversion for the pair
        pair = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){y0, y1}, bf16x2));
      }
      if (EAGER) {
        amax = nan_max(amax, nan_max(fabsf(to_f32_16<F16>(pair & 0xFFFFu)), fabsf(to_f32_16<F16>(pair >> 16))));
      } else {
        amax = nan_max(amax, nan_max(fabsf(y0), fabsf(y1)));
      }
      yb[p][j >> 1] = pair;
    }
  }

  // NaN propagates through the absmax and the floor, as in torch's amax and clamp (a row holding inf or NaN)
  amax = wave_nan_max(amax);
  if (WPR > 1) {
    if (lane == 0) s_amax[wave] = amax;
    __syncthreads();
    amax = nan_max(nan_max(s_amax[0], s_amax[1]), nan_max(s_amax[2], s_amax[3]));
  }
  const float xsv = nan_max(amax / 127.0f, 1e-30f);
  const bool finite_row = __builtin_isfinite(amax);  // uniform: every y and the scale finite
  if (lane == 0 && wr == 0) xs[row] = xsv;
  float s = F16 ? round_f16(xsv) : round_bf16(xsv);
  if (s == 0.0f) s = F16 ? 6.103515625e-05f : 1.1754943508222875e-38f;
  // bf16: bf16(y * fl(1/s)) == bf16(fl(y / s)) for bf16 y and every scale this kernel forms (>= bf16(1e-30));
  // f16: the level is the same (both checked exhaustively on the CPU)
  const float rs = 1.0f / s;

  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int p = 0; p < NPASS; ++p) {
    const int b = (p * WPR + wr) * 4 + g;
    if (b >= nb) continue;
    uint32_t packed[4];
    if (!finite_row) {
      // a row with inf or NaN (rare): y * (1/s) is NaN where the reference's y / s is NaN (inf / inf, NaN), and a
      // NaN quotient converts to level 0 (torch's and numpy's float -> int8 conversion on the reference's host)
#pragma unroll
      for (int w4 = 0; w4 < 4; ++w4) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = w4 * 4 + e;
          const float y = to_f32_16<F16>((yb[p][j >> 1] >> ((j & 1) * 16)) & 0xFFFFu);
          const float t = round16<F16>(fp32_round_point(y * rs));
          const float r = t != t ? 0.0f : __builtin_amdgcn_fmed3f(__builtin_rintf(t), -128.0f, 127.0f);
          word |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xFFu) << (8 * e);
        }
        packed[w4] = word;
      }
    } else if (F16) {
      // f16: round_f16(fl(y * fl(1/s))) can differ from round_f16(fl(y / s)) only between f16 subnormals (|t| <
      // 2^-14), never in the level (checked exhaustively on the CPU); clamp and rint as below.
      uint32_t lv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float y = to_f32_16<F16>((yb[p][j >> 1] >> ((j & 1) * 16)) & 0xFFFFu);
        const float t = __builtin_amdgcn_fmed3f(round_f16(fp32_round_point(y * rs)), -128.0f, 127.0f);
        lv[j] = __float_as_uint(fp32_round_point(t + 12582912.0f));
      }
#pragma unroll
      for (int w4 = 0; w4 < 4; ++w4)
        packed[w4] = __builtin_amdgcn_perm(lv[4 * w4 + 1], lv[4 * w4], 0x0c0c0400u) |
                     __builtin_amdgcn_perm(lv[4 * w4 + 3], lv[4 * w4 + 2], 0x04000c0cu);
    } else {
      // Two elements per word: t = fl(y * fl(1/s)), one packed RNE conversion to bf16 for the pair, clamp, then
      // rint by adding 1.5 * 2^23 (an integer in [2^23, 2^24): its low byte is the two's-complement level).
      // Clamping before the rounding gives the same integer: the bounds are integers exact in bf16 and both
      // roundings are monotone.  A NaN stays NaN through the clamp and the add, and its low byte is 0 (the low 16
      // bits of a widened bf16 are 0), the level the integer conversion gives it.
      uint32_t lv[16];
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        const uint32_t wv = yb[p][h];
        const float t0 = fp32_round_point(__uint_as_float(wv << 16) * rs);
        const float t1 = fp32_round_point(__uint_as_float(wv & 0xFFFF0000u) * rs);
        const uint32_t tb = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){t0, t1}, bf16x2));
        const float r0 = __builtin_amdgcn_fmed3f(__uint_as_float(tb << 16), -128.0f, 127.0f);
        const float r1 = __builtin_amdgcn_fmed3f(__uint_as_float(tb & 0xFFFF0000u), -128.0f, 127.0f);
        lv[2 * h] = __float_as_uint(fp32_round_point(r0 + 12582912.0f));
        lv[2 * h + 1] = __float_as_uint(fp32_round_point(r1 + 12582912.0f));
      }
#pragma unroll
      for (int w4 = 0; w4 < 4; ++w4)
        packed[w4] = __builtin_amdgcn_perm(lv[4 * w4 + 1], lv[4 * w4], 0x0c0c0400u) |
                     __builtin_amdgcn_perm(lv[4 * w4 + 3], lv[4 * w4 + 2], 0x04000c0cu);
    }
    __builtin_nontemporal_store(u32x4{packed[0], packed[1], packed[2], packed[3]},
                                reinterpret_cast<u32x4*>(qr + b * 256 + l * 16));
  }
}

// ------------------------------------------------------------------------------------------------ generic path
// One 256-thread workgroup per row; the row is processed in chunks of 1024 staged in LDS as float64 and
// transformed stage by stage.  Two sweeps: absmax, then quantise (or store the rounded rotation).
template <int DT>
__device__ __forceinline__ float load_x(const void* x, int64_t idx) {
  if (DT == H3K_F32) return static_cast<const float*>(x)[idx];
  const uint32_t bits = static_cast<const uint16_t*>(x)[idx];
  return DT == H3K_F16 ? f16_to_f32(bits) : bf16_to_f32(bits);
}
template <int DT>
__device__ __forceinline__ float round_dt(float f) {
  if (DT == H3K_F32) return f;
  return DT == H3K_F16 ? round_f16(f) : round_bf16(f);
}

template <int DT, bool EAGER, bool ROTATE_ONLY>
__global__ __launch_bounds__(256) void rot_generic_kernel(const void* __restrict__ x, int64_t rows, int k, int64_t ldx,
                                                          int log2, int8_t* __restrict__ q, int64_t ldq,
                                                          float* __restrict__ xs, void* __restrict__ y, int64_t ldy) {
  __shared__ double buf[1024];
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  const int t = threadIdx.x;
  const double scale = rot_scale(log2);
  float amax = 0.0f, s = 1.0f;

  for (int sweep = ROTATE_ONLY ? 1 : 0; sweep < 2; ++sweep) {
    for (int c0 = 0; c0 < k; c0 += 1024) {
      const int n = min(1024, k - c0);
      __syncthreads();
      for (int e = t; e < n; e += 256) buf[e] = static_cast<double>(load_x<DT>(x, row * ldx + c0 + e));
      __syncthreads();
      int S = 1;
      for (int d = 0; d < log2 / 2; ++d, S *= 4) {  // radix-4 stages over bit pairs, from the bottom
        const int base = (t / S) * 4 * S + (t % S);
        if (base < n) h4(buf[base], buf[base + S], buf[base + 2 * S], buf[base + 3 * S]);
        __syncthreads();
      }
      if (log2 & 1) {  // the H2 stage on the top bit
        for (int u = t; u < n / 2; u += 256) {
          const int base = (u / S) * 2 * S + (u % S);
          h2(buf[base], buf[base + S]);
        }
        __syncthreads();
      }
      for (int e = t; e < n; e += 256) {
        const float y32 = static_cast<float>(buf[e] * scale);
        const float yr = round_dt<DT>(y32);
        if (sweep == 0) {
          amax = nan_max(amax, fabsf(EAGER ? yr : y32));
        } else if (ROTATE_ONLY) {
          if (DT == H3K_F32) {
            static_cast<float*>(y)[row * ldy + c0 + e] = yr;
          } else {
            const uint32_t bits = DT == H3K_F16 ? f32_to_f16_bits(y32) : f32_to_bf16_bits(y32);
            static_cast<uint16_t*>(y)[row * ldy + c0 + e] = static_cast<uint16_t>(bits);
          }
        } else {
          float tq = (DT == H3K_F32) ? (yr / s) : round_dt<DT>(fp32_round_point(yr / s));
          tq = tq != tq ? 0.0f : __builtin_amdgcn_fmed3f(__builtin_rintf(tq), -128.0f, 127.0f);  // NaN -> level 0
          q[row * ldq + c0 + e] = static_cast<int8_t>(static_cast<int>(tq));
        }
      }
    }
    if (sweep == 0) {
      amax = wave_nan_max(amax);
      if ((t & 63) == 0) red[t >> 6] = amax;
      __syncthreads();
      amax = nan_max(nan_max(red[0], red[1]), nan_max(red[2], red[3]));
      const float xsv = nan_max(amax / 127.0f, 1e-30f);
      if (t == 0) xs[row] = xsv;
      s = round_dt<DT>(xsv);
      if (s == 0.0f) s = DT == H3K_F16 ? 6.103515625e-05f : 1.1754943508222875e-38f;
    }
  }
}

// ------------------------------------------------------------------------------------------------ host side
template <int NPASS, int WPR, bool F16, bool EAGER, int ACT = kActNone, int ROT = 256>
static void launch256(const void* x, int64_t rows, int k, int64_t ldx, int hshift, int64_t hstride, int8_t* q,
                      int64_t ldq, float* xs, hipStream_t st, const uint16_t* lut) {
  const dim3 grid(static_cast<unsigned>((rows + (4 / WPR) - 1) / (4 / WPR)));
  hipLaunchKernelGGL((rotquant256_kernel<NPASS, WPR, F16, EAGER, ACT, ROT>), grid, dim3(256), 0, st,
                     static_cast<const uint16_t*>(x), rows, k, ldx, hshift, hstride, q, ldq, xs, lut);
}

constexpr int kRqSplitAbove = 8;  // rows longer than this many passes of one wavefront are split over four

// blocks of 256 -> (passes, wavefronts per row); passes 0 when the row is too long for the fast kernel.  Few rows
// (under 2048) are also split, to put more wavefronts on the chip.
static void rq_plan(int blocks, int64_t rows, int& npass, int& wpr) {
  static const int buckets[] = {1, 2, 3, 4, 5, 6, 7, 8};
  wpr = ((blocks + 3) / 4 > kRqSplitAbove || (rows < 2048 && blocks > 4)) ? 4 : 1;
  const int need = (blocks + 4 * wpr - 1) / (4 * wpr);
  npass = 0;
  for (int b : buckets)
    if (b >= need) {
      npass = b;
      break;
    }
}

template <bool F16, bool EAGER, int ACT = kActNone, int ROT = 256>
static bool dispatch256(int npass, int wpr, const void* x, int64_t rows, int k, int64_t ldx, int hshift,
                        int64_t hstride, int8_t* q, int64_t ldq, float* xs, hipStream_t st,
                        const uint16_t* lut = nullptr) {
  switch (npass * 8 + wpr) {
#define H3K_CASE(P, W)      \
  case P * 8 + W:           \
    launch256<P, W, F16, EAGER, ACT, ROT>(x, rows, k, ldx, hshift, hstride, q, ldq, xs, st, lut); \
    return true;
    H3K_CASE(1, 1) H3K_CASE(2, 1) H3K_CASE(3, 1) H3K_CASE(4, 1) H3K_CASE(5, 1) H3K_CASE(6, 1) H3K_CASE(7, 1)
    H3K_CASE(8, 1) H3K_CASE(1, 4) H3K_CASE(2, 4) H3K_CASE(3, 4) H3K_CASE(4, 4) H3K_CASE(5, 4) H3K_CASE(6, 4)
    H3K_CASE(7, 4) H3K_CASE(8, 4)
#undef H3K_CASE
    default:
      return false;
  }
}

static int check_rot_args(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int rot) {
  if (x_dtype != H3K_BF16 && x_dtype != H3K_F16 && x_dtype != H3K_F32)
    return fail(H3K_EINVAL, "activations must be bf16, f16 or f32 (dtype code %d)", x_dtype);
  if (rot < 4 || rot > 1024 || (rot & (rot - 1)))
    return fail(H3K_EINVAL, "rotation block must be a power of 2 in [4, 1024], got %d", rot);
  if (rows < 0 || k <= 0 || k % rot) return fail(H3K_EINVAL, "k=%lld must be a positive multiple of the rotation block %d", (long long)k, rot);
  if (k > (1 << 30)) return fail(H3K_EINVAL, "k=%lld too large", (long long)k);
  if (ldx < k) return fail(H3K_EINVAL, "ldx=%lld < k=%lld", (long long)ldx, (long long)k);
  if (rows > 0 && x == nullptr) return fail(H3K_EINVAL, "x is NULL");
  return H3K_OK;
}

static int log2_of(int rot) {
  int l = 0;
  while (rot > 1) {
    rot >>= 1;
    ++l;
  }
  return l;
}

}  // namespace h3k

using namespace h3k;

extern "C" int h3k_rotate_quant(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int rot, int mode,
                                int8_t* q, int64_t ldq, float* xs, void* stream) {
  int rc = check_rot_args(x, x_dtype, rows, k, ldx, rot);
  if (rc) return rc;
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (ldq < k) return fail(H3K_EINVAL, "ldq=%lld < k=%lld", (long long)ldq, (long long)k);
  if (rows == 0) return H3K_OK;
  if (!q || !xs) return fail(H3K_EINVAL, "q/xs is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool eager = mode == H3K_MODE_EAGER;
  const int es = x_dtype == H3K_F32 ? 4 : 2;
  int np = 0, wpr = 1;
  if (k <= (int64_t)256 * 128) rq_plan(static_cast<int>(k / 256), rows, np, wpr);
  const bool fast = (rot == 256 || rot == 128) && x_dtype != H3K_F32 && aligned(x, 16) && (ldx * es) % 16 == 0 &&
                    aligned(q, 16) && ldq % 16 == 0 && np > 0 && k % 256 == 0;
  if (fast) {
    const int kk = static_cast<int>(k);
    bool ok;
#define H3K_RQ(F, E, R) dispatch256<F, E, kActNone, R>(np, wpr, x, rows, kk, ldx, 31, 0, q, ldq, xs, st)
    if (rot == 256) {
      if (x_dtype == H3K_F16) ok = eager ? H3K_RQ(true, true, 256) : H3K_RQ(true, false, 256);
      else ok = eager ? H3K_RQ(false, true, 256) : H3K_RQ(false, false, 256);
    } else {
      if (x_dtype == H3K_F16) ok = eager ? H3K_RQ(true, true, 128) : H3K_RQ(true, false, 128);
      else ok = eager ? H3K_RQ(false, true, 128) : H3K_RQ(false, false, 128);
    }
#undef H3K_RQ
    if (!ok) return fail(H3K_EINVAL, "no fast rotation kernel for k=%lld", (long long)k);
    return check_launch("rotquant256");
  }
  const dim3 grid(static_cast<unsigned>(rows));
  const int l2 = log2_of(rot), kk = static_cast<int>(k);
#define H3K_GEN(DT, E) \
  hipLaunchKernelGGL((rot_generic_kernel<DT, E, false>), grid, dim3(256), 0, st, x, rows, kk, ldx, l2, q, ldq, xs, nullptr, 0)
  if (x_dtype == H3K_BF16) {
    if (eager) H3K_GEN(H3K_BF16, true); else H3K_GEN(H3K_BF16, false);
  } else if (x_dtype == H3K_F16) {
    if (eager) H3K_GEN(H3K_F16, true); else H3K_GEN(H3K_F16, false);
  } else {
    if (eager) H3K_GEN(H3K_F32, true); else H3K_GEN(H3K_F32, false);
  }
#undef H3K_GEN
  return check_launch("rot_generic(quant)");
}

extern "C" int h3k_rotate_quant_heads(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                                      int head_dim, int64_t head_stride, int rot, int mode, int8_t* q, int64_t ldq,
                                      float* xs, void* stream) {
  if (x_dtype != H3K_BF16 && x_dtype != H3K_F16 && x_dtype != H3K_F32)
    return fail(H3K_EINVAL, "activations must be bf16, f16 or f32 (dtype code %d)", x_dtype);
  if (rows < 0 || ldx < head_dim) return fail(H3K_EINVAL, "rows=%lld, ldx=%lld < head_dim=%d", (long long)rows,
                                              (long long)ldx, head_dim);
  if (x_dtype == H3K_F32 || rot != 256)
    return fail(H3K_EINVAL, "head-major rows take bf16/f16 activations and rotation 256 (dtype %d, rot %d)", x_dtype, rot);
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (head_dim < 16 || (head_dim & (head_dim - 1)) || k % head_dim || k <= 0 || k % 256)
    return fail(H3K_EINVAL, "head_dim=%d must be a power of two >= 16 dividing k=%lld (a multiple of 256)", head_dim,
                (long long)k);
  if (head_stride < rows * ldx) return fail(H3K_EINVAL, "head_stride < rows * ldx (heads overlap)");
  if (ldq < k) return fail(H3K_EINVAL, "ldq=%lld < k=%lld", (long long)ldq, (long long)k);
  if (rows == 0) return H3K_OK;
  if (!x || !q || !xs) return fail(H3K_EINVAL, "x/q/xs is NULL");
  if (!aligned(x, 16) || (ldx * 2) % 16 || (head_stride * 2) % 16 || !aligned(q, 16) || ldq % 16)
    return fail(H3K_EINVAL, "x / q and their strides must be 16-byte aligned");
  int np = 0, wpr = 1;
  if (k <= (int64_t)256 * 128) rq_plan(static_cast<int>(k / 256), rows, np, wpr);
  if (np == 0) return fail(H3K_EINVAL, "k=%lld too long for head-major rows", (long long)k);
  int hshift = 0;
  while ((1 << hshift) < head_dim) ++hshift;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool eager = mode == H3K_MODE_EAGER;
  const int kk = static_cast<int>(k);
  bool ok;
  if (x_dtype == H3K_F16)
    ok = eager ? dispatch256<true, true>(np, wpr, x, rows, kk, ldx, hshift, head_stride, q, ldq, xs, st)
               : dispatch256<true, false>(np, wpr, x, rows, kk, ldx, hshift, head_stride, q, ldq, xs, st);
  else
    ok = eager ? dispatch256<false, true>(np, wpr, x, rows, kk, ldx, hshift, head_stride, q, ldq, xs, st)
               : dispatch256<false, false>(np, wpr, x, rows, kk, ldx, hshift, head_stride, q, ldq, xs, st);
  if (!ok) return fail(H3K_EINVAL, "no fast rotation kernel for k=%lld", (long long)k);
  return check_launch("rotquant256(heads)");
}

// The device's GELU table of the dtype, filled on first use: the fill kernel runs on the caller's stream, which is
// then synchronised once, so that kernels on other streams never read a partly filled table.  A stream under graph
// capture cannot be synchronised: until the table exists such calls evaluate tanhf in the kernel instead (the
// same values).  nullptr means "evaluate in the kernel".
static const uint16_t* gelu_table(bool f16, hipStream_t st) {
  static std::mutex mu;
  static const uint16_t* ready[64][2] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (ready[dev][f16]) return ready[dev][f16];
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  uint16_t* base = nullptr;
  if (hipGetSymbolAddress(reinterpret_cast<void**>(&base), HIP_SYMBOL(g_gelu_lut)) != hipSuccess) return nullptr;
  if (f16) hipLaunchKernelGGL(gelu_lut_kernel<true>, dim3(256), dim3(256), 0, st);
  else hipLaunchKernelGGL(gelu_lut_kernel<false>, dim3(256), dim3(256), 0, st);
  // peek, not get: an error pending from earlier work stays for the entry point's own launch check to report
  if (hipPeekAtLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return nullptr;
  ready[dev][f16] = base + (f16 ? 65536 : 0);
  return ready[dev][f16];
}

extern "C" int h3k_rotate_quant_act(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int act,
                                    int rot, int mode, int8_t* q, int64_t ldq, float* xs, void* stream) {
  if (act != kActSwiglu && act != kActGeluTanh) return fail(H3K_EINVAL, "act must be 1 (swiglu) or 2 (gelu_tanh), got %d", act);
  if (x_dtype != H3K_BF16 && x_dtype != H3K_F16)
    return fail(H3K_EINVAL, "activation-fused rows take bf16 or f16 inputs (dtype code %d)", x_dtype);
  if (rot != 256) return fail(H3K_EINVAL, "activation-fused rows take rotation 256, got %d", rot);
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (rows < 0 || k <= 0 || k % 256) return fail(H3K_EINVAL, "k=%lld must be a positive multiple of 256", (long long)k);
  const int64_t width = act == kActSwiglu ? 2 * k : k;
  if (ldx < width) return fail(H3K_EINVAL, "ldx=%lld < input width %lld", (long long)ldx, (long long)width);
  if (ldq < k) return fail(H3K_EINVAL, "ldq=%lld < k=%lld", (long long)ldq, (long long)k);
  int np = 0, wpr = 1;
  if (k <= (int64_t)256 * 128) rq_plan(static_cast<int>(k / 256), rows, np, wpr);
  if (np == 0) return fail(H3K_EINVAL, "k=%lld too long for the activation-fused kernel", (long long)k);
  if (rows == 0) return H3K_OK;
  if (!x || !q || !xs) return fail(H3K_EINVAL, "x/q/xs is NULL");
  if (!aligned(x, 16) || (ldx * 2) % 16 || !aligned(q, 16) || ldq % 16)
    return fail(H3K_EINVAL, "x / q and their row strides must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool eager = mode == H3K_MODE_EAGER, f16 = x_dtype == H3K_F16;
  const int kk = static_cast<int>(k);
  bool ok;
  // bf16 only: at 12602 x 13824 the table took the kernel from 312 to 216 us; f16's finer codes spread the lookups
  // over far more of the table, and it ran 316 against 312 us
  const uint16_t* lut = act == kActGeluTanh && !f16 ? gelu_table(false, st) : nullptr;
#define H3K_ACT(F, E, A) dispatch256<F, E, A>(np, wpr, x, rows, kk, ldx, 31, 0, q, ldq, xs, st, lut)
  if (act == kActSwiglu)
    ok = f16 ? (eager ? H3K_ACT(true, true, kActSwiglu) : H3K_ACT(true, false, kActSwiglu))
             : (eager ? H3K_ACT(false, true, kActSwiglu) : H3K_ACT(false, false, kActSwiglu));
  else
    ok = f16 ? (eager ? H3K_ACT(true, true, kActGeluTanh) : H3K_ACT(true, false, kActGeluTanh))
             : (eager ? H3K_ACT(false, true, kActGeluTanh) : H3K_ACT(false, false, kActGeluTanh));
#undef H3K_ACT
  if (!ok) return fail(H3K_EINVAL, "no fast rotation kernel for k=%lld", (long long)k);
  return check_launch("rotquant256(act)");
}

extern "C" int h3k_rotate(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int rot, void* y,
                          int64_t ldy, void* stream) {
  int rc = check_rot_args(x, x_dtype, rows, k, ldx, rot);
  if (rc) return rc;
  if (ldy < k) return fail(H3K_EINVAL, "ldy=%lld < k=%lld", (long long)ldy, (long long)k);
  if (rows == 0) return H3K_OK;
  if (!y) return fail(H3K_EINVAL, "y is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
  const int l2 = log2_of(rot), kk = static_cast<int>(k);
  if (x_dtype == H3K_BF16)
    hipLaunchKernelGGL((rot_generic_kernel<H3K_BF16, false, true>), grid, dim3(256), 0, st, x, rows, kk, ldx, l2,
                       nullptr, 0, nullptr, y, ldy);
  else if (x_dtype == H3K_F16)
    hipLaunchKernelGGL((rot_generic_kernel<H3K_F16, false, true>), grid, dim3(256), 0, st, x, rows, kk, ldx, l2,
                       nullptr, 0, nullptr, y, ldy);
  else
    hipLaunchKernelGGL((rot_generic_kernel<H3K_F32, false, true>), grid, dim3(256), 0, st, x, rows, kk, ldx, l2,
                       nullptr, 0, nullptr, y, ldy);
  return check_launch("rot_generic(rotate)");
}
