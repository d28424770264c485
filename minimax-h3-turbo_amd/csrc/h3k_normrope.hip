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

// The attention prologue of the block in one pass over the qkv projection: per token s and head h, read the three
// head rows of qkv [tokens, 3 * heads * D] (q | k | v), apply the norm + rotation above to q and k (the same
// arithmetic in the same order, so the results are bit-identical to qk_norm_rope_kernel), and write q, k, v in the
// head-major layout [heads, tokens, D] that the attention kernel reads (out + h * head_stride + s * D).
//
// A 32-lane half-wavefront owns one head row.  It loads the row with one 2J-byte access per lane (lane l holds
// elements J*l .. J*l+J-1), redistributes it through a private 256-byte LDS row to the partial-sum assignment
// l + 32 j, and gathers the results back the same way for one 2J-byte store per lane.  The 8 half-wavefronts of a
// workgroup take 8 consecutive tokens of one head, so each output head gets 8 * D contiguous elements per
// workgroup and head step; a workgroup walks HPB heads of one of q / k / v.
template <int J>
struct VecOf;
template <>
struct VecOf<1> { typedef uint16_t T; };
template <>
struct VecOf<2> { typedef uint32_t T; };
template <>
struct VecOf<4> { typedef uint2 T; };
template <>
struct VecOf<8> { typedef uint4 T; };

// Head rows per half-wavefront, their loads issued together: at 12602 tokens x 40 heads x 128 (rotary half 48 / 64)
// 8 ran 168 / 157 us, 4 ran 171 / 167 us, and one head at a time (each load behind the previous head's LDS
// round trips) 368 / 383 us.
constexpr int kSplitHPB = 8;

template <int J>
__global__ __launch_bounds__(256) void qkv_split_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int64_t ldqkv, int64_t tokens, int heads, int half, const float* __restrict__ wq,
    const float* __restrict__ wk, const float* __restrict__ cosv, const float* __restrict__ sinv, int64_t ldcs,
    float eps, uint16_t* __restrict__ qo, uint16_t* __restrict__ ko, uint16_t* __restrict__ vo, int64_t head_stride) {
  constexpr int D = 32 * J;
  typedef typename VecOf<J>::T V;
  __shared__ __attribute__((aligned(16))) uint16_t s_row[8][2][D];  // per half-wavefront: input row, output row
  const int hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 8 + hw;
  const int part = blockIdx.z;  // 0 q, 1 k, 2 v
  if (t >= tokens) return;      // whole half-wavefronts leave; nothing below synchronises across them
  const uint16_t* xrow = qkv + t * ldqkv + static_cast<int64_t>(part) * heads * D;
  uint16_t* orow = (part == 0 ? qo : (part == 1 ? ko : vo)) + t * D;
  uint16_t* in = s_row[hw][0];
  uint16_t* outr = s_row[hw][1];
  const float* w = part == 0 ? wq : wk;
  const float* cr = cosv + t * ldcs;
  const float* sr = sinv + t * ldcs;

  // The head rows of this block step are loaded together, so their latencies overlap; the per-lane norm weights
  // and rotary factors do not depend on the head and are read once.
  const int h0 = blockIdx.y * kSplitHPB;
  const int nh = min(kSplitHPB, heads - h0);
  V raw[kSplitHPB];
#pragma unroll
  for (int i = 0; i < kSplitHPB; ++i)
    if (i < nh) raw[i] = *reinterpret_cast<const V*>(xrow + static_cast<int64_t>(h0 + i) * D + J * l);
  if (part == 2) {
#pragma unroll
    for (int i = 0; i < kSplitHPB; ++i)
      if (i < nh) *reinterpret_cast<V*>(orow + static_cast<int64_t>(h0 + i) * head_stride + J * l) = raw[i];
    return;
  }
  float we[J], wp[J], cs[J], sn[J];
  int pe[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = l + 32 * j;
    pe[j] = e < half ? e + half : (e < 2 * half ? e - half : -1);
    we[j] = w[e];
    wp[j] = pe[j] >= 0 ? w[pe[j]] : 0.0f;
    const int ri = e < half ? e : pe[j];  // the rotary index of the pair (e, pe)
    cs[j] = pe[j] >= 0 ? cr[ri] : 0.0f;
    sn[j] = pe[j] >= 0 ? sr[ri] : 0.0f;
  }

#pragma unroll
  for (int i = 0; i < kSplitHPB; ++i) {
    if (i >= nh) break;
    V* dst = reinterpret_cast<V*>(orow + static_cast<int64_t>(h0 + i) * head_stride + J * l);
    wave_lds_sync();  // the previous head's reads of this row are done
    *reinterpret_cast<V*>(in + J * l) = raw[i];
    wave_lds_sync();
    float v[J], pv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = l + 32 * j;
      v[j] = bf16_to_f32(in[e]);
      pv[j] = pe[j] >= 0 ? bf16_to_f32(in[pe[j]]) : 0.0f;
    }
    float partial = fp32_round_point(v[0] * v[0]);
#pragma unroll
    for (int j = 1; j < J; ++j) partial = partial + fp32_round_point(v[j] * v[j]);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) partial = partial + __shfl_down(partial, off, 32);
    const float total = __shfl(partial, 0, 32);
    const float r = 1.0f / sqrtf(fp32_round_point(fp32_round_point(total / static_cast<float>(D)) + eps));
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = l + 32 * j;
      const float n = round_bf16(fp32_round_point(fp32_round_point(v[j] * r) * we[j]));
      float o = n;
      if (pe[j] >= 0) {
        const float np = round_bf16(fp32_round_point(fp32_round_point(pv[j] * r) * wp[j]));
        if (e < half) {
          o = fp32_round_point(n * cs[j]) - fp32_round_point(np * sn[j]);
        } else {
          o = fp32_round_point(np * sn[j]) + fp32_round_point(n * cs[j]);
        }
      }
      outr[e] = static_cast<uint16_t>(f32_to_bf16_bits(o));
    }
    wave_lds_sync();
    *dst = *reinterpret_cast<const V*>(outr + J * l);
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

extern "C" int h3k_qkv_split_norm_rope(const void* qkv, int64_t ldqkv, int64_t tokens, int heads, int head_dim,
                                       const float* wq, const float* wk, const float* cos, const float* sin,
                                       int64_t ldcs, int half, float eps, void* q_out, void* k_out, void* v_out,
                                       int64_t head_stride, void* stream) {
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(H3K_EINVAL, "head_dim=%d must be 32, 64, 128 or 256", head_dim);
  if (half < 0 || 2 * half > head_dim) return fail(H3K_EINVAL, "rotary half=%d exceeds head_dim/2", half);
  if (tokens < 0 || heads <= 0) return fail(H3K_EINVAL, "bad tokens/heads");
  if (ldqkv < 3 * static_cast<int64_t>(heads) * head_dim || ldcs < half || head_stride < tokens * head_dim)
    return fail(H3K_EINVAL, "strides smaller than the rows (ldqkv >= 3*heads*head_dim, head_stride >= tokens*head_dim)");
  if (tokens == 0) return H3K_OK;
  if (!qkv || !wq || !wk || !q_out || !k_out || !v_out || (half > 0 && (!cos || !sin)))
    return fail(H3K_EINVAL, "NULL pointer");
  const size_t vb = static_cast<size_t>(head_dim) / 16;  // bytes per lane access (head_dim / 32 elements)
  if (!aligned(qkv, vb) || (ldqkv * 2) % vb || !aligned(q_out, vb) || !aligned(k_out, vb) || !aligned(v_out, vb) ||
      (head_stride * 2) % vb)
    return fail(H3K_EINVAL, "qkv / outputs / strides must be aligned to head_dim/16 bytes");
  if (tokens > (int64_t(1) << 31) * 8) return fail(H3K_EINVAL, "too many tokens");
  const dim3 grid(static_cast<unsigned>((tokens + 7) / 8), static_cast<unsigned>((heads + kSplitHPB - 1) / kSplitHPB), 3);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(qkv);
  uint16_t *qo = static_cast<uint16_t*>(q_out), *ko = static_cast<uint16_t*>(k_out), *vo = static_cast<uint16_t*>(v_out);
  switch (head_dim / 32) {
#define H3K_SP(J)                                                                                                  \
  case J:                                                                                                          \
    hipLaunchKernelGGL((qkv_split_norm_rope_kernel<J>), grid, dim3(256), 0, st, x, ldqkv, tokens, heads, half, wq, \
                       wk, cos, sin, ldcs, eps, qo, ko, vo, head_stride);                                          \
    break;
    H3K_SP(1) H3K_SP(2) H3K_SP(4) H3K_SP(8)
#undef H3K_SP
  }
  return check_launch("qkv_split_norm_rope");
}
