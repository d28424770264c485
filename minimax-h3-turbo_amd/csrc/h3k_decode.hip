// int4 codebook indices -> exact int8 grid (reference h3turbo/h3/qlinear.py:157-204):
//   w8[n, k] = clamp(rint_half_even(f32(codebook[nib(n, k)]) * f32(s_rel[n, k / group])), -127, 127)
// nib(n, 2j) is the LOW nibble of q[n, j]; a NaN product (NaN scale byte) decodes to 0 like the reference's
// nan_to_num'd pair table.  HBM-bound: each thread turns 8 packed bytes into 16 levels (one 16-byte store).
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

template <int SD, bool SMALL_GROUP>
__global__ __launch_bounds__(256) void decode_w4_kernel(const uint8_t* __restrict__ q, int64_t ldq,
                                                        const void* __restrict__ s_rel, int64_t lds,
                                                        const float* __restrict__ cb, int64_t n, int k, int group,
                                                        int8_t* __restrict__ w8, int64_t ldw) {
  __shared__ float s_cb[16];
  if (threadIdx.x < 16) s_cb[threadIdx.x] = cb[threadIdx.x];
  __syncthreads();
  const int chunks = k >> 4;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= n * chunks) return;
  const int64_t row = t / chunks;
  const int c = static_cast<int>(t - row * chunks);
  const uint2 pk = *reinterpret_cast<const uint2*>(q + row * ldq + c * 8);
  const int64_t srow = row * lds;
  float sc = 0.0f;
  if (!SMALL_GROUP) sc = load_scale<SD>(s_rel, srow + (c * 16) / group);
  uint32_t out[4];
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4) {
    const uint32_t word = w4 < 2 ? pk.x : pk.y;
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = w4 * 4 + e;  // element within the 16-chunk
      const uint32_t byte = (word >> (8 * ((i >> 1) & 3))) & 0xFFu;
      const uint32_t nib = (i & 1) ? (byte >> 4) : (byte & 0xFu);
      const float s = SMALL_GROUP ? load_scale<SD>(s_rel, srow + (c * 16 + i) / group) : sc;
      o |= level(s_cb[nib], s) << (8 * e);
    }
    out[w4] = o;
  }
  *reinterpret_cast<uint4*>(w8 + row * ldw + c * 16) = make_uint4(out[0], out[1], out[2], out[3]);
}

template <int SD>
static void launch_decode(const void* q, int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int64_t n, int k,
                          int group, int8_t* w8, int64_t ldw, hipStream_t st) {
  const int64_t threads = n * (k / 16);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (group < 16)
    hipLaunchKernelGGL((decode_w4_kernel<SD, true>), grid, dim3(256), 0, st, static_cast<const uint8_t*>(q), ldq, s_rel,
                       lds, cb, n, k, group, w8, ldw);
  else
    hipLaunchKernelGGL((decode_w4_kernel<SD, false>), grid, dim3(256), 0, st, static_cast<const uint8_t*>(q), ldq,
                       s_rel, lds, cb, n, k, group, w8, ldw);
}

}  // namespace h3k

using namespace h3k;

extern "C" int h3k_decode_w4(const void* q, int64_t ldq, const void* s_rel, int s_dtype, int64_t lds,
                             const float* codebook, int64_t n, int64_t k, int group, int8_t* w8, int64_t ldw,
                             void* stream) {
  if (s_dtype != H3K_FP8E4M3 && s_dtype != H3K_F16 && s_dtype != H3K_BF16 && s_dtype != H3K_F32)
    return fail(H3K_EINVAL, "s_rel dtype code %d unsupported (fp8e4m3/f16/bf16/f32)", s_dtype);
  if (group < 4 || k <= 0 || k % 16 || k % group || ((16 % group) && (group % 16)))
    return fail(H3K_EINVAL,
                "K=%lld must be divisible by 16 and group_size=%d; group_size >= 4 dividing 16 or a multiple of 16",
                (long long)k, group);
  if (n < 0 || k > (1 << 30)) return fail(H3K_EINVAL, "bad n/k");
  if (ldq < k / 2 || lds < k / group || ldw < k) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (n == 0) return H3K_OK;
  if (!q || !s_rel || !codebook || !w8) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(q, 8) || ldq % 8) return fail(H3K_EINVAL, "q must be 8-byte aligned with an 8-byte multiple row stride");
  if (!aligned(w8, 16) || ldw % 16) return fail(H3K_EINVAL, "w8 must be 16-byte aligned with a 16-byte multiple row stride");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kk = static_cast<int>(k);
  switch (s_dtype) {
    case H3K_FP8E4M3: launch_decode<H3K_FP8E4M3>(q, ldq, s_rel, lds, codebook, n, kk, group, w8, ldw, st); break;
    case H3K_F16: launch_decode<H3K_F16>(q, ldq, s_rel, lds, codebook, n, kk, group, w8, ldw, st); break;
    case H3K_BF16: launch_decode<H3K_BF16>(q, ldq, s_rel, lds, codebook, n, kk, group, w8, ldw, st); break;
    default: launch_decode<H3K_F32>(q, ldq, s_rel, lds, codebook, n, kk, group, w8, ldw, st); break;
  }
  return check_launch("decode_w4");
}
