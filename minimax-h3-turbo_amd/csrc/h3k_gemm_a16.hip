// W4A8 linear with unquantised activations ("a16", reference h3turbo/h3/qlinear.py:407-424, _TorchRunner._a16):
//   y[m, n] = sum_k xr[m, k] * level[n, k]        fp32 accumulation; xr = the rotated activation in its 16-bit dtype
//   out     = round_out(fp32(y * s_ch[n]) + bias[n])                      bias optional, fp32
// The int8 levels are exact in bf16 and f16 (at most 8 significant bits), so the GEMM runs on the 16-bit MFMA
// (v_mfma_f32_32x32x16_bf16 / _f16) on (xr, levels) with fp32 accumulators: the weights are never rounded and the
// output is rounded once, as in the reference's tensor-core path.
//
// Tile 128 x 128 per workgroup, 4 wavefronts as 2 x 2, each 64 x 64 = 2 x 2 blocks of 32 x 32.  K advances 64 per
// stage through a 2-stage LDS ring: the activations as loaded, the int8 levels widened to the activation dtype on
// the way in (16 bytes of int8 -> 32 bytes).  The next stage's global loads are in flight in registers while this
// stage computes.  Weights are the MFMA's first operand, so each lane's accumulators hold one output row (4
// consecutive columns per group).  Rows past M or N read a clamped row and are not stored; K is a multiple of 16
// and chunks past K read as zeros.
#include "h3k_common.hpp"

namespace h3k {
namespace a16 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int ROWB = BK * 2;         // bytes of one LDS row (64 16-bit values)
constexpr int STAGE = (BM + BN) * ROWB;  // 32 KiB: activations, then levels

// 16-byte chunk c of LDS row r, XOR-swizzled over 8 chunks: the fragment reads of 32 consecutive rows at one chunk
// spread over all banks.
__device__ __forceinline__ int chunk_at(int r, int c) { return r * ROWB + ((c ^ (r & 7)) << 4); }

// 4 int8 levels (one word) -> 4 16-bit values in the activation dtype, exact.
template <bool F16>
__device__ __forceinline__ uint2 widen4(uint32_t w) {
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f = static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xFFu));
    h[i] = F16 ? static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)))
               : (__float_as_uint(f) >> 16);  // |level| <= 128: exact in bf16, low bits zero
  }
  return make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

template <bool F16, int ODT>
__global__ __launch_bounds__(256, 2) void gemm_a16_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                         const int8_t* __restrict__ W, int64_t ldw,
                                                         const float* __restrict__ sch, const float* __restrict__ bias,
                                                         int M, int N, int K, void* __restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int KT = (K + BK - 1) / BK;

  // loads of one stage: activations 128 rows x 8 chunks (4 per thread), levels 128 rows x 4 chunks of 16 (2 per
  // thread; each becomes 2 LDS chunks)
  u32x4 ra[4], rw[2];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = i * 256 + tid, r = id >> 3, c = id & 7;
      const int k = kt * BK + c * 8;
      const int row = min(m0 + r, M - 1);
      ra[i] = k < K ? *reinterpret_cast<const u32x4*>(A + static_cast<int64_t>(row) * lda + k) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = i * 256 + tid, r = id >> 2, c = id & 3;
      const int k = kt * BK + c * 16;
      const int row = min(n0 + r, N - 1);
      rw[i] = k < K ? *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(row) * ldw + k) : u32x4{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
    uint8_t* sa = smem + buf * STAGE;
    uint8_t* sw = sa + BM * ROWB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = i * 256 + tid, r = id >> 3, c = id & 7;
      *reinterpret_cast<u32x4*>(sa + chunk_at(r, c)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = i * 256 + tid, r = id >> 2, c = id & 3;
      const uint2 a = widen4<F16>(rw[i][0]), b = widen4<F16>(rw[i][1]), d = widen4<F16>(rw[i][2]),
                  e = widen4<F16>(rw[i][3]);
      *reinterpret_cast<u32x4*>(sw + chunk_at(r, 2 * c)) = u32x4{a.x, a.y, b.x, b.y};
      *reinterpret_cast<u32x4*>(sw + chunk_at(r, 2 * c + 1)) = u32x4{d.x, d.y, e.x, e.y};
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 31, fh = lane >> 5;  // fragment row within a block, k half (8 values) within 16
  for (int kt = 0; kt < KT; ++kt) {
    const bool more = kt + 1 < KT;
    if (more) load(kt + 1);
    const uint8_t* sa = smem + (kt & 1) * STAGE;
    const uint8_t* sw = sa + BM * ROWB;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + fh;
      u32x4 fa[2], fw[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const u32x4*>(sa + chunk_at(wm * 64 + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < 2; ++j) fw[j] = *reinterpret_cast<const u32x4*>(sw + chunk_at(wn * 64 + j * 32 + fr, c));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (F16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, fw[j]),
                                                               __builtin_bit_cast(f16x8, fa[i]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fw[j]),
                                                                __builtin_bit_cast(bf16x8, fa[i]), acc[i][j], 0, 0, 0);
        }
    }
    if (more) store((kt + 1) & 1);  // the other buffer: every wave finished reading it before the last barrier
    __syncthreads();
  }

  // epilogue: lane owns output row m, columns n = base + g * 8 + fh * 4 + e of each block
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 64 + i * 32 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + j * 32 + g * 8 + fh * 4;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int nn = min(n + e, N - 1);
          float v = fp32_round_point(acc[i][j][g * 4 + e] * sch[nn]);
          if (bias) v = fp32_round_point(v + bias[nn]);
          y[e] = v;
        }
        const int64_t off = static_cast<int64_t>(m) * ldo + n;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= N) break;
          if (ODT == H3K_F32) static_cast<float*>(out)[off + e] = y[e];
          else if (ODT == H3K_F16) static_cast<uint16_t*>(out)[off + e] = static_cast<uint16_t>(f32_to_f16_bits(y[e]));
          else static_cast<uint16_t*>(out)[off + e] = static_cast<uint16_t>(f32_to_bf16_bits(y[e]));
        }
      }
    }
  }
}

template <bool F16, int ODT>
static void launch(const void* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sch, const float* bias,
                   int m, int n, int k, void* out, int64_t ldo, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((n + BN - 1) / BN), static_cast<unsigned>((m + BM - 1) / BM));
  hipLaunchKernelGGL((gemm_a16_kernel<F16, ODT>), grid, dim3(256), 0, st, static_cast<const uint16_t*>(a), lda, w, ldw,
                     sch, bias, m, n, k, out, ldo);
}

}  // namespace a16
}  // namespace h3k

using namespace h3k;

extern "C" int h3k_gemm_a16(const void* a, int a_dtype, int64_t lda, const int8_t* w8, int64_t ldw, const float* s_ch,
                            const float* bias, int64_t m, int64_t n, int64_t k, void* out, int out_dtype, int64_t ldo,
                            void* stream) {
  if (a_dtype != H3K_BF16 && a_dtype != H3K_F16) return fail(H3K_EINVAL, "a16 activations must be bf16 or f16");
  if (out_dtype != H3K_BF16 && out_dtype != H3K_F16 && out_dtype != H3K_F32)
    return fail(H3K_EINVAL, "out dtype code %d unsupported", out_dtype);
  if (m < 0 || n < 0 || k <= 0 || k % 16 || m > (1 << 30) || n > (1 << 30) || k > (1 << 24))
    return fail(H3K_EINVAL, "bad a16 GEMM shape m=%lld n=%lld k=%lld (k a positive multiple of 16)", (long long)m,
                (long long)n, (long long)k);
  if (lda < k || ldw < k || ldo < n) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (m == 0 || n == 0) return H3K_OK;
  if (!a || !w8 || !s_ch || !out) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(a, 16) || lda % 8 || !aligned(w8, 16) || ldw % 16)
    return fail(H3K_EINVAL, "activation and level rows must be 16-byte aligned");
  if ((m + a16::BM - 1) / a16::BM > 65535) return fail(H3K_EINVAL, "m=%lld too large for one launch", (long long)m);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
#define H3K_A16(F, O) a16::launch<F, O>(a, lda, w8, ldw, s_ch, bias, mi, ni, ki, out, ldo, st)
  if (a_dtype == H3K_F16) {
    if (out_dtype == H3K_BF16) H3K_A16(true, H3K_BF16);
    else if (out_dtype == H3K_F16) H3K_A16(true, H3K_F16);
    else H3K_A16(true, H3K_F32);
  } else {
    if (out_dtype == H3K_BF16) H3K_A16(false, H3K_BF16);
    else if (out_dtype == H3K_F16) H3K_A16(false, H3K_F16);
    else H3K_A16(false, H3K_F32);
  }
#undef H3K_A16
  return check_launch("gemm_a16");
}
