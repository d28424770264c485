// Per-head RMSNorm + split-half rotary embedding of q and k, in place, bf16 (reference h3turbo/h3/layout.py:309-355,
// norm_rope_ with impl "torch", the numerics of the fused q/k kernel the reference reproduces).  Per head row x[D]:
//   part[l]  = sum_{j < D/32} fp32(x[32 j + l])^2, j in order (each square rounded to fp32, then each add)
//   total    = halving tree over the 32 parts: part[l] += part[l + off], off = 16, 8, 4, 2, 1
//   r        = 1 / sqrt(total / D + eps)               (correctly rounded division and square root)
//   n[e]     = bf16((x[e] * r) * w[e])
//   e < half           : out = bf16(n[e] * c[e] - n[e + half] * s[e])
//   half <= e < 2 half : out = bf16(n[e - half] * s[e - half] + n[e] * c[e - half])
//   e >= 2 half        : out = n[e]
// with every fp32 product and sum rounded separately (no contraction).  One 32-lane half-wavefront per head row:
// lane l owns elements l + 32 j, which is exactly the partial-sum assignment, so the tree runs on lane shuffles.
// A lane also reads the rotation partners of its elements; all loads of a row precede its stores (one wavefront).
#include "h3k_common.hpp"

namespace h3k {

template <int J>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(uint16_t* __restrict__ q, int64_t ldq, uint16_t* __restrict__ k,
                                                           int64_t ldk, int64_t tokens, int heads, int half,
                                                           const float* __restrict__ wq, const float* __restrict__ wk,
                                                           const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                           int64_t ldcs, float eps) {
  constexpr int D = 32 * J;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  const int64_t rows = tokens * heads * 2;
  if (row >= rows) return;
  const int l = threadIdx.x & 31;
  const int64_t t = row / (2 * heads);
  const int rem = static_cast<int>(row - t * 2 * heads);
  const bool is_k = rem >= heads;
  const int h = is_k ? rem - heads : rem;
  uint16_t* x = (is_k ? k + t * ldk : q + t * ldq) + static_cast<int64_t>(h) * D;
  const float* w = is_k ? wk : wq;
  const float* cr = cosv + t * ldcs;
  const float* sr = sinv + t * ldcs;

  float v[J], pv[J];
  int pe[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = l + 32 * j;
    v[j] = bf16_to_f32(x[e]);
    pe[j] = e < half ? e + half : (e < 2 * half ? e - half : -1);
    pv[j] = pe[j] >= 0 ? bf16_to_f32(x[pe[j]]) : 0.0f;
  }
  float part = fp32_round_point(v[0] * v[0]);
#pragma unroll
  for (int j = 1; j < J; ++j) part = part + fp32_round_point(v[j] * v[j]);
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) part = part + __shfl_down(part, off, 32);
  const float total = __shfl(part, 0, 32);
  const float r = 1.0f / sqrtf(fp32_round_point(fp32_round_point(total / static_cast<float>(D)) + eps));

#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = l + 32 * j;
    const float n = round_bf16(fp32_round_point(fp32_round_point(v[j] * r) * w[e]));
    float o = n;
    if (pe[j] >= 0) {
      const int p = pe[j];
      const float np = round_bf16(fp32_round_point(fp32_round_point(pv[j] * r) * w[p]));
      if (e < half) {  // lo = n, hi = np
        o = fp32_round_point(n * cr[e]) - fp32_round_point(np * sr[e]);
      } else {  // lo = np (element e - half), hi = n
        o = fp32_round_point(np * sr[p]) + fp32_round_point(n * cr[p]);
      }
    }
    x[e] = static_cast<uint16_t>(f32_to_bf16_bits(o));
  }
}

}  // namespace h3k

using namespace h3k;

extern "C" int h3k_qk_norm_rope(void* q, int64_t ldq, void* k, int64_t ldk, int64_t tokens, int heads, int head_dim,
                                const float* wq, const float* wk, const float* cos, const float* sin, int64_t ldcs,
                                int half, float eps, void* stream) {
  if (head_dim % 32 || head_dim < 32 || head_dim > 256)
    return fail(H3K_EINVAL, "head_dim=%d must be a multiple of 32 in [32, 256]", head_dim);
  if (half < 0 || 2 * half > head_dim) return fail(H3K_EINVAL, "rotary half=%d exceeds head_dim/2", half);
  if (tokens < 0 || heads <= 0) return fail(H3K_EINVAL, "bad tokens/heads");
  if (ldq < static_cast<int64_t>(heads) * head_dim || ldk < static_cast<int64_t>(heads) * head_dim || ldcs < half)
    return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (tokens == 0) return H3K_OK;
  if (!q || !k || !wq || !wk || (half > 0 && (!cos || !sin))) return fail(H3K_EINVAL, "NULL pointer");
  const int64_t rows = tokens * heads * 2;
  const dim3 grid(static_cast<unsigned>((rows + 7) / 8));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* qp = static_cast<uint16_t*>(q);
  uint16_t* kp = static_cast<uint16_t*>(k);
  switch (head_dim / 32) {
#define H3K_NR(J)                                                                                                  \
  case J:                                                                                                          \
    hipLaunchKernelGGL((qk_norm_rope_kernel<J>), grid, dim3(256), 0, st, qp, ldq, kp, ldk, tokens, heads, half, wq, \
                       wk, cos, sin, ldcs, eps);                                                                   \
    break;
    H3K_NR(1) H3K_NR(2) H3K_NR(3) H3K_NR(4) H3K_NR(5) H3K_NR(6) H3K_NR(7) H3K_NR(8)
#undef H3K_NR
  }
  return check_launch("qk_norm_rope");
}
