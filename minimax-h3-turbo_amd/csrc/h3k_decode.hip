// int4 codebook indices -> exact int8 grid (reference h3turbo/h3/qlinear.py:157-204):
//   w8[n, k] = clamp(rint_half_even(f32(codebook[nib(n, k)]) * f32(s_rel[n, k / group])), -127, 127)
// nib(n, 2j) is the LOW nibble of q[n, j]; a NaN product (NaN scale byte) decodes to 0 like the reference's
// nan_to_num'd pair table.  HBM-bound: each thread turns 8 packed bytes into 16 levels (one 16-byte store), or for
// groups of 32 or more 32 levels through a 16-entry byte table per scale (decode_w4_lut_kernel); fp8 scales of
// other groups from 16 up read the tables of all 256 scale bytes from LDS (decode_w4_fp8tab_kernel).
#include "h3k_w4.hpp"

namespace h3k {

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

// fp8 scales with groups of 16 (or odd multiples of 16), where a thread's 16 levels share one scale: an e4m3 scale
// has 256 byte values, so the workgroup first builds the 16-entry table of every one (4 KiB of LDS, entry e byte i =
// level(codebook[i], fp8(e)), the per-element function) and each of its threads then decodes kFp8TabReps chunks of
// 16 levels, each through the table of its scale byte with byte permutes.  Consecutive threads take consecutive
// chunks, so every pass of the workgroup loads 2 KiB and stores 4 KiB contiguous (within a row).
constexpr int kFp8TabReps = 8;

__global__ __launch_bounds__(256) void decode_w4_fp8tab_kernel(const uint8_t* __restrict__ q, int64_t ldq,
                                                               const uint8_t* __restrict__ s_rel, int64_t lds,
                                                               const float* __restrict__ cb, int64_t n, int k,
                                                               int group, int8_t* __restrict__ w8, int64_t ldw) {
  __shared__ __attribute__((aligned(16))) uint32_t tab[256 * 4];
  {
    const float s = fp8e4m3fn_to_f32(threadIdx.x);  // blockDim.x == 256: one entry per thread
    uint32_t w4[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      w4[w] = level(cb[4 * w], s) | (level(cb[4 * w + 1], s) << 8) | (level(cb[4 * w + 2], s) << 16) |
              (level(cb[4 * w + 3], s) << 24);
    *reinterpret_cast<u32x4*>(tab + threadIdx.x * 4) = u32x4{w4[0], w4[1], w4[2], w4[3]};
  }
  __syncthreads();  // nothing returns before it
  const int chunks = k >> 4;
  const int64_t total = n * chunks;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * kFp8TabReps) + threadIdx.x;
#pragma unroll
  for (int r = 0; r < kFp8TabReps; ++r) {
    const int64_t t = base + r * 256;
    if (t >= total) break;
    const int64_t row = t / chunks;
    const int c = static_cast<int>(t - row * chunks);
    const uint2 pk = *reinterpret_cast<const uint2*>(q + row * ldq + c * 8);
    const uint32_t sbyte = s_rel[row * lds + (c * 16) / group];  // a u8: the table index stays below 256
    const u32x4 e = *reinterpret_cast<const u32x4*>(tab + sbyte * 4);
    const uint32_t lut[4] = {e[0], e[1], e[2], e[3]};
    uint32_t o0, o1, o2, o3;
    lut_decode_word(lut, pk.x, o0, o1);
    lut_decode_word(lut, pk.y, o2, o3);
    *reinterpret_cast<uint4*>(w8 + row * ldw + c * 16) = make_uint4(o0, o1, o2, o3);
  }
}

// The 4-word byte table of a scale that SH aligned lanes of a quad share (1, 2 or 4): lane j of the SH holds words
// j * 4 / SH .. + 4 / SH; quad permutes hand every lane all four.  Every lane of the SH must be active.
template <int SH>
__device__ __forceinline__ void share_lut(const uint32_t (&mine)[4 / SH], uint32_t (&lut)[4]) {
  if constexpr (SH == 1) {
#pragma unroll
    for (int w = 0; w < 4; ++w) lut[w] = mine[w];
  } else if constexpr (SH == 2) {  // quad_perm [0,0,2,2] / [1,1,3,3]
    lut[0] = __builtin_amdgcn_mov_dpp(mine[0], 0xA0, 0xF, 0xF, false);
    lut[1] = __builtin_amdgcn_mov_dpp(mine[1], 0xA0, 0xF, 0xF, false);
    lut[2] = __builtin_amdgcn_mov_dpp(mine[0], 0xF5, 0xF, 0xF, false);
    lut[3] = __builtin_amdgcn_mov_dpp(mine[1], 0xF5, 0xF, 0xF, false);
  } else {  // quad_perm [w,w,w,w]
    lut[0] = __builtin_amdgcn_mov_dpp(mine[0], 0x00, 0xF, 0xF, false);
    lut[1] = __builtin_amdgcn_mov_dpp(mine[0], 0x55, 0xF, 0xF, false);
    lut[2] = __builtin_amdgcn_mov_dpp(mine[0], 0xAA, 0xF, 0xF, false);
    lut[3] = __builtin_amdgcn_mov_dpp(mine[0], 0xFF, 0xF, 0xF, false);
  }
}

// The SH-lane share of a scale's table: words j * 4 / SH .. of level(codebook[.], s).
template <int SH>
__device__ __forceinline__ void build_shared_lut(const float* __restrict__ cb, float s, int j, uint32_t (&lut)[4]) {
  constexpr int NW = 4 / SH;
  uint32_t mine[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int w = j * NW + i;
    mine[i] = level(cb[4 * w], s) | (level(cb[4 * w + 1], s) << 8) | (level(cb[4 * w + 2], s) << 16) |
              (level(cb[4 * w + 3], s) << 24);
  }
  share_lut<SH>(mine, lut);
}

// Groups of 32 or more: a thread owns 32 consecutive levels of one row (16 packed bytes in, 32 bytes out, so a
// wavefront's loads and stores are contiguous) that share one scale.  The scale's 16 possible levels form a byte
// table in 4 registers (byte c of word w = level(codebook[4w + c], s)); the SH lanes of a quad that share the
// scale each compute 4/SH of its words and broadcast them with DPP quad permutes.  A nibble becomes its level
// with byte permutes: one v_perm_b32 over entries 0-7, one over entries 8-15, and a third that picks between
// them on the nibble's bit 3.  The levels are the same values the per-element path computes.
template <int SD, int SH>
__global__ __launch_bounds__(256) void decode_w4_lut_kernel(const uint8_t* __restrict__ q, int64_t ldq,
                                                            const void* __restrict__ s_rel, int64_t lds,
                                                            const float* __restrict__ cb, int n, int k, int group,
                                                            int8_t* __restrict__ w8, int64_t ldw) {
  static_assert(SH == 1 || SH == 2 || SH == 4, "lanes sharing a scale");
  const int chunks = k >> 5;  // a multiple of SH (host), so whole quads stay in one row and one scale group
  const int t = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (t >= n * chunks) return;  // whole quads; n * chunks < 2^31 (host)
  const int row = t / chunks;
  const int c = t - row * chunks;
  const u32x4 pk = *reinterpret_cast<const u32x4*>(q + static_cast<int64_t>(row) * ldq + c * 16);
  const float s = load_scale<SD>(s_rel, static_cast<int64_t>(row) * lds + (c * 32) / group);
  uint32_t lut[4];
  build_shared_lut<SH>(cb, s, t & (SH - 1), lut);
  uint32_t o[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t dlo = lut_lookup(lut, pk[w] & 0x07070707u, (pk[w] >> 1) & 0x04040404u);  // even k: low nibbles
    const uint32_t dhi = lut_lookup(lut, (pk[w] >> 4) & 0x07070707u, (pk[w] >> 5) & 0x04040404u);  // odd k
    o[2 * w] = __builtin_amdgcn_perm(dhi, dlo, 0x05010400u);      // lo0 hi0 lo1 hi1
    o[2 * w + 1] = __builtin_amdgcn_perm(dhi, dlo, 0x07030602u);  // lo2 hi2 lo3 hi3
  }
  int8_t* dst = w8 + static_cast<int64_t>(row) * ldw + c * 32;
  *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<u32x4*>(dst + 16) = u32x4{o[4], o[5], o[6], o[7]};
}

// The same levels written in the packed layout of the large-shape GEMM (h3k_gemm_w8p.hip): 64-byte K-steps t of
// 32-row blocks b (N padded to a multiple of 256 rows), block (t, b) 2 KiB at (t * NBP + b) * 2048 as two 1 KiB MFMA
// fragments in which lane l holds row 32b + (l & 31), bytes 64t + 32(l >> 5) + 16h .. + 16.  A thread owns one row's
// 32 consecutive levels (16 packed bytes in, the two 16-byte halves out).  A workgroup takes K-steps 4T .. 4T + 3 of
// one 32-row block: eight consecutive threads own a row's 128 packed bytes there, so every load instruction reads 8
// whole 128-byte lines and every store writes 8 runs of 128 bytes (8 rows' 16 bytes, consecutive in a fragment).
// Workgroups of one K-step each would split each line of the weight between workgroups far apart in time, and it
// was fetched again.  Rows past n (the padding) are written as zeros.  GK: 0 for groups that are multiples of 32
// (one scale per thread, its 16 levels as a byte table; SH = 4 or 2 for groups that are multiples of 128 or 64,
// where the quad's or pair's lanes, which hold k = 256T + 32j .. and so share a scale, each build 4 / SH words of
// it and exchange them), 1 for group 16 (two tables), 2 for groups 4 and 8 (levels computed per element).  The
// early returns below take whole sharing groups: a row's 8 lanes share its row, and with K a multiple of 128
// (SH = 4) or the lanes of a pair sharing t (SH = 2) a group's lanes are past the last K-step together.
template <int SD, int GK, int SH>
__global__ __launch_bounds__(256) void decode_w4_packed_kernel(const uint8_t* __restrict__ q, int64_t ldq,
                                                               const void* __restrict__ s_rel, int64_t lds,
                                                               const float* __restrict__ cb, int n, int nbp,
                                                               int group, int8_t* __restrict__ wp, int kt) {
  // fp8 scales of group 16: the workgroup's table of all 256 scale bytes (entry e: build_lut_fast at fp8(e)), built
  // before any thread returns; a thread's two tables are then two 16-byte LDS reads
  constexpr bool kTab = SD == H3K_FP8E4M3 && GK == 1;
  __shared__ __attribute__((aligned(16))) uint32_t tab[kTab ? 256 * 4 : 4];
  if constexpr (kTab) {
    float cbv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) cbv[i] = cb[i];
    uint32_t w4[4];
    build_lut_fast(cbv, all_finite(cbv), fp8e4m3fn_to_f32(threadIdx.x), w4);  // blockDim.x == 256
    *reinterpret_cast<u32x4*>(tab + threadIdx.x * 4) = u32x4{w4[0], w4[1], w4[2], w4[3]};
    __syncthreads();
  }
  const int b = static_cast<int>(blockIdx.x % static_cast<unsigned>(nbp));
  const int j = static_cast<int>(threadIdx.x & 7);  // 32-level chunk of the row within the 4 K-steps
  const int t = static_cast<int>(blockIdx.x / static_cast<unsigned>(nbp)) * 4 + (j >> 1);
  if (t >= kt) return;  // the last K-step group of a K-step count not a multiple of 4 (no cross-lane work below)
  const int l = (j & 1) * 32 + static_cast<int>(threadIdx.x >> 3);  // the fragment lane: row l & 31, half l >> 5
  const int64_t bt = static_cast<int64_t>(t) * nbp + b;
  const int row = b * 32 + (l & 31);
  const int k0 = t * 64 + (l >> 5) * 32;  // first of this thread's 32 levels
  int8_t* dst = wp + bt * 2048 + l * 16;
  if (row >= n) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(dst + 1024) = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const u32x4 pk = *reinterpret_cast<const u32x4*>(q + static_cast<int64_t>(row) * ldq + k0 / 2);
  const int64_t srow = static_cast<int64_t>(row) * lds;
  uint32_t o[8];
  if constexpr (GK == 2) {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t v = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = w * 4 + e;  // level index within the 32
        const uint32_t byte = (pk[i >> 3] >> (8 * ((i >> 1) & 3))) & 0xFFu;
        const uint32_t nib = (i & 1) ? (byte >> 4) : (byte & 0xFu);
        v |= level(cb[nib], load_scale<SD>(s_rel, srow + (k0 + i) / group)) << (8 * e);
      }
      o[w] = v;
    }
  } else if (kTab) {
    const uint8_t* sbytes = static_cast<const uint8_t*>(s_rel) + srow + k0 / 16;  // u8: indexes stay below 256
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 e = *reinterpret_cast<const u32x4*>(tab + static_cast<uint32_t>(sbytes[h]) * 4);
      const uint32_t lut[4] = {e[0], e[1], e[2], e[3]};
      lut_decode_word(lut, pk[2 * h], o[4 * h], o[4 * h + 1]);
      lut_decode_word(lut, pk[2 * h + 1], o[4 * h + 2], o[4 * h + 3]);
    }
  } else if (GK == 0 && SH > 1) {
    uint32_t lut[4];
    build_shared_lut<SH>(cb, load_scale<SD>(s_rel, srow + k0 / group), j & (SH - 1), lut);
#pragma unroll
    for (int w = 0; w < 4; ++w) lut_decode_word(lut, pk[w], o[2 * w], o[2 * w + 1]);
  } else {
    float cbv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) cbv[i] = cb[i];
    const bool cb_finite = all_finite(cbv);
    uint32_t lut[4];
    build_lut_fast(cbv, cb_finite, load_scale<SD>(s_rel, srow + k0 / group), lut);
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // 4 packed bytes -> 8 levels
      if (GK == 1 && w == 2) build_lut_fast(cbv, cb_finite, load_scale<SD>(s_rel, srow + (k0 + 16) / group), lut);
      lut_decode_word(lut, pk[w], o[2 * w], o[2 * w + 1]);
    }
  }
  *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<u32x4*>(dst + 1024) = u32x4{o[4], o[5], o[6], o[7]};
}

template <int SD>
static void launch_decode_packed(const void* q, int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int64_t n,
                                 int k, int group, int8_t* wp, hipStream_t st) {
  const int nbp = static_cast<int>((n + 255) / 256 * 8);
  const int kt = k / 64;
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(nbp) * ((kt + 3) / 4)));  // < 2^32 (host checks)
  const uint8_t* qb = static_cast<const uint8_t*>(q);
  const int nn = static_cast<int>(n);
#define H3K_DP(GK, SH)                                                                                              \
  hipLaunchKernelGGL((decode_w4_packed_kernel<SD, GK, SH>), grid, dim3(256), 0, st, qb, ldq, s_rel, lds, cb, nn, nbp,  \
                     group, wp, kt)
  if (group % 128 == 0) H3K_DP(0, 4);
  else if (group % 64 == 0) H3K_DP(0, 2);
  else if (group % 32 == 0) H3K_DP(0, 1);
  else if (group == 16) H3K_DP(1, 1);
  else H3K_DP(2, 1);
#undef H3K_DP
}

template <int SD>
static void launch_decode(const void* q, int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int64_t n, int k,
                          int group, int8_t* w8, int64_t ldw, hipStream_t st) {
  const int sh = group % 128 == 0 ? 4 : (group % 64 == 0 ? 2 : 1);
  if (group % 32 == 0 && n * (k / 32) < (int64_t(1) << 31) - 256 && aligned(q, 16) && ldq % 16 == 0) {
    const dim3 g(static_cast<unsigned>((n * (k / 32) + 255) / 256));
    const int nn = static_cast<int>(n);
#define H3K_DL(SH)                                                                                                  \
    hipLaunchKernelGGL((decode_w4_lut_kernel<SD, SH>), g, dim3(256), 0, st, static_cast<const uint8_t*>(q), ldq,   \
                       s_rel, lds, cb, nn, k, group, w8, ldw)
    if (sh == 4) H3K_DL(4); else if (sh == 2) H3K_DL(2); else H3K_DL(1);
#undef H3K_DL
    return;
  }
  const int64_t threads = n * (k / 16);
  if (SD == H3K_FP8E4M3 && group >= 16) {
    const dim3 g(static_cast<unsigned>((threads + 256 * kFp8TabReps - 1) / (256 * kFp8TabReps)));
    hipLaunchKernelGGL(decode_w4_fp8tab_kernel, g, dim3(256), 0, st, static_cast<const uint8_t*>(q), ldq,
                       static_cast<const uint8_t*>(s_rel), lds, cb, n, k, group, w8, ldw);
    return;
  }
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

extern "C" int h3k_decode_w4_packed(const void* q, int64_t ldq, const void* s_rel, int s_dtype, int64_t lds,
                                    const float* codebook, int64_t n, int64_t k, int group, int8_t* w8p,
                                    void* stream) {
  if (s_dtype != H3K_FP8E4M3 && s_dtype != H3K_F16 && s_dtype != H3K_BF16 && s_dtype != H3K_F32)
    return fail(H3K_EINVAL, "s_rel dtype code %d unsupported (fp8e4m3/f16/bf16/f32)", s_dtype);
  if (group < 4 || k <= 0 || k % 64 || k % group || ((16 % group) && (group % 16)))
    return fail(H3K_EINVAL,
                "K=%lld must be divisible by 64 and group_size=%d; group_size >= 4 dividing 16 or a multiple of 16",
                (long long)k, group);
  // The grid has (N' * K) / 8192 workgroups of 256 threads; its work-item count must stay below 2^32.
  if (n < 0 || n > (1 << 30) || k > (1 << 30) || (n + 255) / 256 * 256 * k >= (int64_t(1) << 37))
    return fail(H3K_EINVAL, "bad n/k");
  if (ldq < k / 2 || lds < k / group) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (n == 0) return H3K_OK;
  if (!q || !s_rel || !codebook || !w8p) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(q, 16) || ldq % 16 || !aligned(w8p, 16))
    return fail(H3K_EINVAL, "q must be 16-byte aligned with a 16-byte multiple row stride, w8p 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kk = static_cast<int>(k);
  switch (s_dtype) {
    case H3K_FP8E4M3: launch_decode_packed<H3K_FP8E4M3>(q, ldq, s_rel, lds, codebook, n, kk, group, w8p, st); break;
    case H3K_F16: launch_decode_packed<H3K_F16>(q, ldq, s_rel, lds, codebook, n, kk, group, w8p, st); break;
    case H3K_BF16: launch_decode_packed<H3K_BF16>(q, ldq, s_rel, lds, codebook, n, kk, group, w8p, st); break;
    default: launch_decode_packed<H3K_F32>(q, ldq, s_rel, lds, codebook, n, kk, group, w8p, st); break;
  }
  return check_launch("decode_w4_packed");
}
