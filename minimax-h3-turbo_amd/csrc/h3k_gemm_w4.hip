// W4A8 GEMM for few token rows (M <= 128) with the int4 weight decoded in registers: the int8 grid never exists in
// HBM (reference h3turbo/h3/qlinear.py:157-204 decode, :236-254 int8 GEMM, :396-405 epilogue, fused).
//
//   acc[m, n] = sum_k a[m, k] * level(n, k)                      exact int32
//   level(n, k) = clamp(rint(codebook[nib(n, k)] * s_rel[n, k / group]), -127, 127)   (NaN product -> 0)
//   ck / eager epilogue and bias exactly as h3k_gemm_a8w8.
//
// Few rows make the op a stream over the packed weight (4 * M int8 ops per weight byte): the kernel reads q, the
// scales and the codebook once and turns them into MFMA operands in registers.
//
// Layout.  A workgroup of 4 wavefronts owns 128 output columns (32 per wavefront) and all M rows (padded to 32 * MB)
// for one slice of K.  A K-step is 64 bytes.  In v_mfma_i32_32x32x32_i8 a lane supplies 16 k of one row, lanes
// 0-31 and 32-63 the two 16-k halves of a 32-k block.  Any permutation of k applied to both operands leaves the dot
// product unchanged, so this kernel hands lane (column c, half h) the 32 consecutive k [64t + 32h, 64t + 32h + 32)
// of its column: 16 packed bytes, one 16-byte load, two fragments (k + [0, 16) and k + [16, 32)).  The A fragments
// follow the same assignment (LDS chunk 2h + s of the 64-byte row).  The lane decodes its 32 levels through the
// scale's byte table (h3k_w4.hpp): groups of 64 or more rebuild the table only where a group starts, group 32 once
// per step, group 16 twice per step.
//
// Latency.  A workgroup owns 8 K-steps (512 k).  It issues all its reads before computing: 8 x 16 bytes of packed
// weight per lane into registers and its whole A slice (XOR-swizzled per step) into LDS, then one barrier; the K loop
// has no barrier and no memory access but its LDS reads (each step's scales are loaded up front too).  blockIdx.y walks the K splits: each adds its exact int32
// partial sums into a zeroed workspace with vector atomics (integer addition: the order does not matter) and a
// second kernel applies the epilogue.  K of 512 or less is one split, with the epilogue fused.
#include "h3k_w4.hpp"

namespace h3k {
namespace w4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;        // K bytes per step
constexpr int kNW = 4;         // wavefronts per workgroup
constexpr int kBN = 32 * kNW;  // output columns per workgroup
constexpr int kMaxM = 128;
constexpr int kSteps = 8;      // K-steps (512 k) per workgroup: one K split

__device__ __forceinline__ int swz(int r, int c) { return r * kBK + ((c ^ ((r >> 1) & 3)) << 4); }

// The epilogue's output dtype and order are runtime arguments: they only act once per output.
__device__ __forceinline__ void store_out(int odt, bool eager, int a, float xv, float sc, float bv, bool has_bias,
                                          void* out, int64_t o) {
  float f = fp32_round_point(eager ? static_cast<float>(a) * fp32_round_point(xv * sc)
                                   : fp32_round_point(static_cast<float>(a) * xv) * sc);
  if (odt == H3K_F32) {
    if (has_bias) f = f + bv;
    static_cast<float*>(out)[o] = f;
  } else if (odt == H3K_F16) {
    f = round_f16(f);
    if (has_bias) f = fp32_round_point(f + bv);
    static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_f16_bits(f));
  } else {
    f = round_bf16(f);
    if (has_bias) f = fp32_round_point(f + bv);
    static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_bf16_bits(f));
  }
}

__device__ __forceinline__ float load_bias(int odt, const void* bias, int n) {
  if (odt == H3K_F32) return static_cast<const float*>(bias)[n];
  if (odt == H3K_F16) return f16_to_f32(static_cast<const uint16_t*>(bias)[n]);
  return bf16_to_f32(static_cast<const uint16_t*>(bias)[n]);
}

// GK: 16 (two scales per lane and step), 32 (one per step), 64 (group a multiple of 64: one per group)
template <int MB, int SD, int GK, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_w4_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ xs, const uint8_t* __restrict__ q,
                                                      int64_t ldq, const void* __restrict__ s_rel, int64_t lds,
                                                      const float* __restrict__ cb, int group,
                                                      const float* __restrict__ sch, const void* __restrict__ bias,
                                                      int M, int N, int K, void* __restrict__ out, int64_t ldo,
                                                      int odt, bool eager, int32_t* __restrict__ ws,
                                                      int32_t* __restrict__ acc_out) {
  constexpr int MP = 32 * MB;
  constexpr int TILE = MP * kBK;                     // one K-step of A in LDS
  constexpr int A_CH = kSteps * MP * (kBK / 16);     // 16-byte chunks of the workgroup's A slice
  constexpr int A_LD = (A_CH + 255) / 256;           // per thread
  __shared__ __attribute__((aligned(16))) int8_t sA[kSteps * TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = blockIdx.x * kBN + wave * 32 + (lane & 31);
  const int kh = lane >> 5;
  const bool nok = col < N;
  const int crow = nok ? col : N - 1;  // out-of-range columns read a valid row; their outputs are dropped
  const uint8_t* qrow = q + static_cast<int64_t>(crow) * ldq + kh * 16;
  const int64_t srow = static_cast<int64_t>(crow) * lds;
  const int KT = K / kBK;
  const int t0 = blockIdx.y * kSteps;
  const int nsteps = min(kSteps, KT - t0);

  // Every memory read of the workgroup's slice goes out before any compute: the packed weight into registers
  // (16 bytes per lane and step), the A slice into LDS.
  u32x4 pk[kSteps];
#pragma unroll
  for (int j = 0; j < kSteps; ++j)
    pk[j] = j < nsteps ? *reinterpret_cast<const u32x4*>(qrow + static_cast<int64_t>(t0 + j) * (kBK / 2))
                       : u32x4{0, 0, 0, 0};
  {
    u32x4 ra[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i;
      const int j = id / (MP * 4), rc = id - j * (MP * 4), r = rc >> 2, c = rc & 3;
      ra[i] = (id < A_CH && j < nsteps && r < M)
                  ? *reinterpret_cast<const u32x4*>(A + static_cast<int64_t>(r) * lda + (t0 + j) * kBK + c * 16)
                  : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i;
      const int j = id / (MP * 4), rc = id - j * (MP * 4), r = rc >> 2, c = rc & 3;
      if (id < A_CH) *reinterpret_cast<u32x4*>(&sA[j * TILE + swz(r, c)]) = ra[i];
    }
  }
  // the scale(s) of each step's 32 k, converted to fp32 (group 16: two per step)
  float sv[kSteps], sv2[kSteps];
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    const int k0 = (t0 + j) * kBK + kh * 32;
    const bool in = j < nsteps;
    if (GK == 16) {
      sv[j] = in ? load_scale<SD>(s_rel, srow + k0 / 16) : 0.0f;
      sv2[j] = in ? load_scale<SD>(s_rel, srow + k0 / 16 + 1) : 0.0f;
    } else if (GK == 32) {
      sv[j] = in ? load_scale<SD>(s_rel, srow + k0 / 32) : 0.0f;
    } else if (j == 0 || ((t0 + j) * kBK) % group == 0) {  // uniform: where a group starts
      sv[j] = in ? load_scale<SD>(s_rel, srow + k0 / group) : 0.0f;
    }
  }
  float cbv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) cbv[i] = cb[i];
  const bool cbf = all_finite(cbv);
  v16i acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = v16i{};
  uint32_t lut[4] = {0, 0, 0, 0}, lut2[4] = {0, 0, 0, 0};
  __syncthreads();

#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    if (j >= nsteps) break;  // uniform
    const int t = t0 + j;  // this lane's 32 k: [64t + 32kh, +32)
    if (GK == 16) {
      build_lut_fast(cbv, cbf, sv[j], lut);
      build_lut_fast(cbv, cbf, sv2[j], lut2);
    } else if (GK == 32) {
      build_lut_fast(cbv, cbf, sv[j], lut);
    } else if (j == 0 || (t * kBK) % group == 0) {  // uniform: groups are multiples of 64
      build_lut_fast(cbv, cbf, sv[j], lut);
    }
    // a lane past N decodes its (valid, clamped) row as is: B row n only reaches output column n, never stored
    v4i bf[2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t lo4, hi4;
      if (GK == 16 && w >= 2) lut_decode_word(lut2, pk[j][w], lo4, hi4);
      else lut_decode_word(lut, pk[j][w], lo4, hi4);
      bf[w >> 1][(w & 1) * 2] = static_cast<int>(lo4);
      bf[w >> 1][(w & 1) * 2 + 1] = static_cast<int>(hi4);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const v4i af = *reinterpret_cast<const v4i*>(&sA[j * TILE + swz(i * 32 + (lane & 31), 2 * kh + s)]);
        acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[s], acc[i], 0, 0, 0);
      }
    }
  }

  // C layout of a 32x32 block: lane l holds column (l % 32); register r holds row (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  if (!nok) return;
  float sc = 0.0f, bv = 0.0f;
  if (!SPLIT) {
    sc = sch[col];
    if (bias) bv = load_bias(odt, bias, col);
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = i * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
      if (m >= M) continue;
      const int a = acc[i][r];
      const int64_t e = static_cast<int64_t>(m) * N + col;
      if (SPLIT) {
        atomicAdd(ws + e, a);
      } else {
        if (acc_out) acc_out[e] = a;
        store_out(odt, eager, a, xs[m], sc, bv, bias != nullptr, out, static_cast<int64_t>(m) * ldo + col);
      }
    }
  }
}

// Up to 32 rows: a workgroup owns 32 output columns and its 4 wavefronts split the workgroup's K range in four;
// each wavefront loads its A fragments (rows x 16 bytes per step, from L2: A is small and shared by every
// workgroup) and its packed weight straight into registers, in chunks of kChunk steps, the next chunk in flight
// while the current one computes.  The four partial sums meet in LDS (a fixed order) and one wavefront per
// quarter of the rows applies the epilogue; only narrow N splits K across workgroups as well (vector atomics
// into the workspace, then the epilogue kernel).
constexpr int kChunk = 4;

// fp8 scales with groups of 16 or 32 take each group's level table from a table of all 256 scale bytes that the
// workgroup builds once in LDS (entry e: the 4 words build_lut_fast gives for scale byte e), one 16-byte LDS read
// per group in place of ~70 VALU.  The scales then travel as their raw bytes.
template <int SD, int GK>
constexpr bool col_scale_table() {
  return SD == H3K_FP8E4M3 && (GK == 16 || GK == 32);
}

template <int MB, int SD, int GK>
struct ColChunk {
  u32x4 pq[kChunk];
  u32x4 pa[kChunk][2 * MB];
  float s1[kChunk], s2[kChunk];
  uint32_t b1[kChunk], b2[kChunk];  // raw fp8 scale bytes (col_scale_table)
};

// Loads of chunk slots past the wavefront's range read its last step (valid) and are never computed; A rows past M
// read row M - 1 and only reach output rows that are never stored.  So no load is predicated.  first, nst and tw0
// are wavefront-uniform (scalar registers).
template <int MB, int SD, int GK>
__device__ __forceinline__ void col_load(ColChunk<MB, SD, GK>& c, int first, int nst, int tw0, const uint8_t* qrow,
                                         const int8_t* const (&arow)[MB], const void* s_rel, int64_t srow, int kh,
                                         int group) {
  const uint8_t* qb = qrow + static_cast<int64_t>(tw0 + first) * (kBK / 2);
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const int off = min(first + j, nst - 1) - first;  // j, except past the range
    c.pq[j] = *reinterpret_cast<const u32x4*>(qb + off * (kBK / 2));
    const int t = tw0 + first + off;
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        c.pa[j][2 * b + s] = *reinterpret_cast<const u32x4*>(arow[b] + static_cast<int64_t>(t) * kBK + s * 16);
    const int k0 = t * kBK + kh * 32;
    if (col_scale_table<SD, GK>()) {
      const uint8_t* sbytes = static_cast<const uint8_t*>(s_rel) + srow;
      c.b1[j] = sbytes[k0 / GK];
      if (GK == 16) c.b2[j] = sbytes[k0 / 16 + 1];
    } else if (GK == 16) {
      c.s1[j] = load_scale<SD>(s_rel, srow + k0 / 16);
      c.s2[j] = load_scale<SD>(s_rel, srow + k0 / 16 + 1);
    } else if (GK == 32) {
      c.s1[j] = load_scale<SD>(s_rel, srow + k0 / 32);
    } else {
      c.s1[j] = load_scale<SD>(s_rel, srow + k0 / group);
    }
  }
}

template <int MB, int SD, int GK>
__device__ __forceinline__ void col_compute(const ColChunk<MB, SD, GK>& c, int first, int nst, int tw0,
                                            const float (&cbv)[16], bool cbf, uint32_t (&lut)[4], uint32_t (&lut2)[4],
                                            v16i (&acc)[MB], int group, const uint32_t* tab) {
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const int i = first + j;
    if (i >= nst) break;  // uniform within the wavefront
    const int t = tw0 + i;
    if (col_scale_table<SD, GK>()) {  // bytes of u8 loads: & 0xFF only states the table's bound
      const u32x4 t1 = *reinterpret_cast<const u32x4*>(tab + (c.b1[j] & 0xFFu) * 4);
#pragma unroll
      for (int w = 0; w < 4; ++w) lut[w] = t1[w];
      if (GK == 16) {
        const u32x4 t2 = *reinterpret_cast<const u32x4*>(tab + (c.b2[j] & 0xFFu) * 4);
#pragma unroll
        for (int w = 0; w < 4; ++w) lut2[w] = t2[w];
      }
    } else if (GK == 16) {
      build_lut_fast(cbv, cbf, c.s1[j], lut);
      build_lut_fast(cbv, cbf, c.s2[j], lut2);
    } else if (GK == 32 || i == 0 || (t * kBK) % group == 0) {
      build_lut_fast(cbv, cbf, c.s1[j], lut);
    }
    // a lane past N decodes its (valid, clamped) row as is: B row n only reaches output column n, never stored
    v4i bf[2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t lo4, hi4;
      if (GK == 16 && w >= 2) lut_decode_word(lut2, c.pq[j][w], lo4, hi4);
      else lut_decode_word(lut, c.pq[j][w], lo4, hi4);
      bf[w >> 1][(w & 1) * 2] = static_cast<int>(lo4);
      bf[w >> 1][(w & 1) * 2 + 1] = static_cast<int>(hi4);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const u32x4 a = c.pa[j][2 * b + s];
        const v4i af = {static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3])};
        acc[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[s], acc[b], 0, 0, 0);
      }
  }
}

template <int MB, int SD, int GK, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_w4_col_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                          const float* __restrict__ xs, const uint8_t* __restrict__ q,
                                                          int64_t ldq, const void* __restrict__ s_rel, int64_t lds,
                                                          const float* __restrict__ cb, int group,
                                                          const float* __restrict__ sch, const void* __restrict__ bias,
                                                          int M, int N, int K, int wsteps, void* __restrict__ out,
                                                          int64_t ldo, int odt, bool eager, int32_t* __restrict__ ws,
                                                          int32_t* __restrict__ acc_out) {
  __shared__ int32_t red[4][MB * 16][64];  // each wavefront's accumulators, register-major
  __shared__ __attribute__((aligned(16))) uint32_t tab[col_scale_table<SD, GK>() ? 256 * 4 : 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar K-range bookkeeping
  const int col = blockIdx.x * 32 + (lane & 31);
  const int kh = lane >> 5;
  const bool nok = col < N;
  const int crow = nok ? col : N - 1;
  const uint8_t* qrow = q + static_cast<int64_t>(crow) * ldq + kh * 16;
  const int64_t srow = static_cast<int64_t>(crow) * lds;
  const int KT = K / kBK;
  const int tw0 = (blockIdx.y * 4 + wave) * wsteps;  // this wavefront's first K-step
  const int nst = max(0, min(wsteps, KT - tw0));
  const int8_t* arow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int r = min(b * 32 + (lane & 31), M - 1);
    arow[b] = A + static_cast<int64_t>(r) * lda + kh * 32;  // lane's k: 64t + 32kh + 16s
  }
  float cbv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) cbv[i] = cb[i];
  const bool cbf = all_finite(cbv);
  v16i acc[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) acc[b] = v16i{};
  uint32_t lut[4] = {0, 0, 0, 0}, lut2[4] = {0, 0, 0, 0};
  if (col_scale_table<SD, GK>()) {  // 256 threads, one entry each; nothing returns before this barrier
    uint32_t w4[4];
    build_lut_fast(cbv, cbf, fp8e4m3fn_to_f32(static_cast<uint32_t>(tid)), w4);
    *reinterpret_cast<u32x4*>(tab + tid * 4) = u32x4{w4[0], w4[1], w4[2], w4[3]};
    __syncthreads();
  }

  ColChunk<MB, SD, GK> c0, c1;
  if (nst > 0) col_load(c0, 0, nst, tw0, qrow, arow, s_rel, srow, kh, group);
  for (int first = 0; first < nst; first += 2 * kChunk) {
    if (first + kChunk < nst) col_load(c1, first + kChunk, nst, tw0, qrow, arow, s_rel, srow, kh, group);
    col_compute(c0, first, nst, tw0, cbv, cbf, lut, lut2, acc, group, tab);
    if (first + 2 * kChunk < nst) col_load(c0, first + 2 * kChunk, nst, tw0, qrow, arow, s_rel, srow, kh, group);
    col_compute(c1, first + kChunk, nst, tw0, cbv, cbf, lut, lut2, acc, group, tab);
  }

#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][b * 16 + r][lane] = acc[b][r];
  __syncthreads();
  if (!nok) return;
  float sc = 0.0f, bv = 0.0f;
  if (!SPLIT) {
    sc = sch[col];
    if (bias) bv = load_bias(odt, bias, col);
  }
  // wavefront w finishes registers [w * 4 * MB, (w + 1) * 4 * MB) of every lane
#pragma unroll
  for (int u = 0; u < 4 * MB; ++u) {
    const int rr = wave * 4 * MB + u;  // register index across the MB blocks
    const int b = rr >> 4, r = rr & 15;
    const int m = b * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
    if (m >= M) continue;
    const int a = red[0][rr][lane] + red[1][rr][lane] + red[2][rr][lane] + red[3][rr][lane];
    const int64_t e = static_cast<int64_t>(m) * N + col;
    if (SPLIT) {
      atomicAdd(ws + e, a);
    } else {
      if (acc_out) acc_out[e] = a;
      store_out(odt, eager, a, xs[m], sc, bv, bias != nullptr, out, static_cast<int64_t>(m) * ldo + col);
    }
  }
}

// ------------------------------------------------------------------------------------------------ 16-row tiles
// Up to 16 rows with K a multiple of 128 and enough columns to fill the chip (gemm_w4_c16_kernel).
//
// v_mfma_i32_16x16x64_i8 takes 16 rows of A per fragment, so one A fragment feeds the two 16-column groups of a
// wavefront's 32 columns.  A super-step is 128 k: lane group g = lane / 16 takes the 32 consecutive k
// [128t + 32g, 128t + 32g + 32) of its column and splits them over the two MFMA sub-steps (k + [0, 16), k + [16, 32));
// its A fragments take the same k of its row (any permutation of k applied to both operands leaves the sums
// unchanged).  So the four lanes of a column share a scale wherever the group spans 128 k (64: pairs of lanes): each
// builds one word (two) of the 16-byte table and they exchange words through ds_bpermute.  The table level is
// clamp(rint(c * s)) with the rounding done by adding 1.5 * 2^23 (the sum is an integer in [2^23, 2^24), its low
// byte the two's-complement level).
//
// Loads.  A workgroup owns 32 columns; its wavefronts split K into contiguous runs of stages (256 k).  A wavefront
// stages its packed weight (32 columns x 128 bytes) and A (16 rows x 256 bytes) in 8 KiB of LDS, loaded as whole
// 128-byte lines (8 lanes per line) through a buffer descriptor, then reads its MFMA fragments back with
// ds_read_b128: the fragment layout touches each line in 64-byte halves, which costs twice the memory requests when
// loaded straight into registers.  The next stage's loads (32 registers per lane) are in flight while this stage
// computes; they go to LDS after its fragment reads.  The lane offsets are fixed; the stage moves in the scalar
// offset.  The wavefronts' partial sums meet in LDS in a fixed order.
constexpr int kSS = 128;           // k per super-step
constexpr int kC16MinTiles = 128;  // fewer 32-column tiles leave the chip idle: the split-K column kernel serves

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                         static_cast<int>(soff), 0));
}

template <int SD>
__device__ __forceinline__ uint32_t bload_scale_bits(rsrc_t r, uint32_t voff, uint32_t soff) {
  if (SD == H3K_FP8E4M3) return __builtin_amdgcn_raw_buffer_load_b8(r, static_cast<int>(voff), static_cast<int>(soff), 0);
  if (SD == H3K_F16 || SD == H3K_BF16)
    return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(voff), static_cast<int>(soff), 0);
  return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

template <int SD>
__device__ __forceinline__ float scale_value(uint32_t bits) {
  if (SD == H3K_FP8E4M3) return fp8e4m3fn_to_f32(bits);
  if (SD == H3K_F16) return f16_to_f32(bits);
  if (SD == H3K_BF16) return bf16_to_f32(bits);
  return __uint_as_float(bits);
}

template <int SD>
constexpr int scale_bytes() {
  return SD == H3K_FP8E4M3 ? 1 : (SD == H3K_F32 ? 4 : 2);
}

// level(c, s) + 1.5 * 2^23 for a finite product: the low byte is the level.
__device__ __forceinline__ uint32_t level_addend(float cbv, float s) {
  const float p = __builtin_amdgcn_fmed3f(fp32_round_point(cbv * s), -127.0f, 127.0f);
  return __float_as_uint(fp32_round_point(p + 12582912.0f));
}

// Table word of codebook entries c[0..3] at scale s (byte i = level(c[i], s)); the NaN-aware form unless every
// product is finite.
__device__ __forceinline__ uint32_t lut_word(const float* c, float s, bool fast) {
  if (fast) {
    const uint32_t b0 = level_addend(c[0], s), b1 = level_addend(c[1], s), b2 = level_addend(c[2], s),
                   b3 = level_addend(c[3], s);
    return __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u) | __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);
  }
  return level(c[0], s) | (level(c[1], s) << 8) | (level(c[2], s) << 16) | (level(c[3], s) << 24);
}

// LDS staging of one wavefront: kStage k of its 32 columns (packed) and of the 16 A rows.  A 16-byte chunk of column
// c (row r) sits at chunk index ch ^ ((c >> 1) & 7) (ch ^ r), so the 16 lanes of one ds_read_b128 pass (same lane
// group, 16 columns or rows) hit 16 different bank groups; the loads choose their global chunk to match.
constexpr int kStage = 256;                  // k per stage: two super-steps, whole 128-byte lines of packed weight
constexpr int kQStage = 32 * kStage / 2;     // 4 KiB
constexpr int kAStage = 16 * kStage;         // 4 KiB
constexpr int kWaveLds = kQStage + kAStage;
constexpr int kC16MaxWaves = 8;              // <= 128 VGPRs: two workgroups of 8 per CU (64 KiB of LDS each)

// GK: 16, 32, 64, 128 (group 128) or 256 (a multiple of 128 above 128: the table is rebuilt where a group starts)
template <int SD, int GK>
__global__ __launch_bounds__(64 * kC16MaxWaves) void gemm_w4_c16_kernel(
    const int8_t* __restrict__ A, int64_t lda, const float* __restrict__ xs, const uint8_t* __restrict__ q, int64_t ldq,
    const void* __restrict__ s_rel, int64_t lds, const float* __restrict__ cb, int group, const float* __restrict__ sch,
    const void* __restrict__ bias, int M, int N, int K, int spw, void* __restrict__ out, int64_t ldo, int odt,
    bool eager, int32_t* __restrict__ acc_out) {
  // fp8 scales with groups of 16 or 32 (a table per group, ~70 VALU each): the tables of all 256 scale bytes are
  // built once per workgroup into 4 KiB of LDS (entry e = the 4 words of scale byte e), and a group's table is one
  // 16-byte LDS read.  Same lut_word on the same operands: the same bytes as building it in place.
  constexpr bool kTab = SD == H3K_FP8E4M3 && (GK == 16 || GK == 32);
  constexpr int kTabBytes = kTab ? 256 * 16 : 0;
  __shared__ __attribute__((aligned(1024))) int8_t smem[kC16MaxWaves * kWaveLds + kTabBytes];
  const int8_t* const tab = smem + kC16MaxWaves * kWaveLds;
  constexpr uint32_t sb = scale_bytes<SD>();
  constexpr int NS = GK == 16 ? 2 : 1;  // scales per lane, column and super-step

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = static_cast<int>(blockDim.x) >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int KS = K / kSS, NSTG = (KS + 1) / 2;
  const int st0 = wave * spw;
  const int nst = max(0, min(spw, NSTG - st0));
  int8_t* const qs = smem + wave * kWaveLds;  // the wavefront's stage: packed weight, then A
  int8_t* const as = qs + kQStage;

  const rsrc_t rq = make_rsrc(q, static_cast<uint32_t>(static_cast<int64_t>(N - 1) * ldq + K / 2));
  const rsrc_t ra = make_rsrc(A, static_cast<uint32_t>(static_cast<int64_t>(M - 1) * lda + K));
  const rsrc_t rs = make_rsrc(s_rel, static_cast<uint32_t>((static_cast<int64_t>(N - 1) * lds + K / group) * sb));
  // load i: packed-weight columns 8i + lane / 8 (8 lanes per 128-byte line), A rows 4i + lane / 16 (16 lanes per
  // 256-byte row); each lane's 16 bytes go to their swizzled LDS chunk.  Columns past N and rows past M are not
  // clamped: their offsets lie past the descriptor's range, the loads return zeros, and those columns and rows only
  // reach outputs that are never stored.
  const uint32_t qoff = static_cast<uint32_t>((static_cast<int64_t>(blockIdx.x) * 32 + (lane >> 3)) * ldq + ((lane & 7) << 4));
  const uint32_t aoff = static_cast<uint32_t>(static_cast<int64_t>(lane >> 4) * lda + ((lane & 15) << 4));
  const uint32_t qstep = static_cast<uint32_t>(8 * ldq), astep = static_cast<uint32_t>(4 * lda);  // per load i
  // LDS chunk of load i: q column c = 8i + lane / 8 at c * 128 + ((lane & 7) ^ ((c >> 1) & 7)) * 16, where
  // (c >> 1) & 7 = 4 (i & 1) + lane / 16; A row r = 4i + lane / 16 at r * 256 + ((lane & 15) ^ r) * 16
  const uint32_t qdst0 = static_cast<uint32_t>((lane >> 3) * 128 + (((lane & 7) ^ (lane >> 4)) << 4));
  const uint32_t qdst1 = static_cast<uint32_t>((lane >> 3) * 128 + (((lane & 7) ^ (4 + (lane >> 4))) << 4));
  const uint32_t adst0 = static_cast<uint32_t>((lane >> 4) * 256 + (((lane & 15) ^ (lane >> 4)) << 4));
  uint32_t soff[2];  // the lane's first scale of its two columns (past N: past the range, zeros)
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const int col = static_cast<int>(blockIdx.x) * 32 + cg * 16 + c16;
    uint32_t sl = 0;
    if (GK == 64) sl = g >> 1;
    else if (GK == 32) sl = g;
    else if (GK == 16) sl = 2 * g;
    soff[cg] = static_cast<uint32_t>((static_cast<int64_t>(col) * lds + sl) * sb);
  }

  constexpr int NCB = GK >= 128 ? 4 : (GK == 64 ? 8 : 16);
  float cbw[NCB];
  const int cb0 = GK >= 128 ? 4 * g : (GK == 64 ? 8 * (g & 1) : 0);
#pragma unroll
  for (int i = 0; i < NCB; ++i) cbw[i] = cb[cb0 + i];
  bool cbw_finite = true;
#pragma unroll
  for (int i = 0; i < NCB; ++i) cbw_finite = cbw_finite && __builtin_isfinite(cbw[i]);
  if (kTab) {
    for (int e = tid; e < 256; e += static_cast<int>(blockDim.x)) {
      const float s = scale_value<SD>(static_cast<uint32_t>(e));
      const bool fast = cbw_finite && __builtin_isfinite(s);
      uint32_t w4[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) w4[w] = lut_word(&cbw[4 * w], s, fast);
      *reinterpret_cast<u32x4*>(smem + kC16MaxWaves * kWaveLds + e * 16) = u32x4{w4[0], w4[1], w4[2], w4[3]};
    }
    __syncthreads();  // every thread of the workgroup reaches it: nothing returns before the main loop
  }
  // ds_bpermute byte addresses of the lanes that build the column's table words
  const uint32_t bp0 = GK >= 128 ? static_cast<uint32_t>(c16 * 4) : static_cast<uint32_t>((c16 + 16 * (g & 2)) * 4);

  v4i acc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
  uint32_t lut[2][4] = {}, lut2[2][4] = {};

  // ---- stage st into registers (whole-line loads) and the scales of its super-steps
  u32x4 rq4[4], ra4[4];
  uint32_t snext[2][2][NS], scur[2][2][NS];  // [super-step][column group][16-k half]
  auto load = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rq4[i] = bload16(rq, qoff, static_cast<uint32_t>(st) * (kStage / 2) + i * qstep);
#pragma unroll
    for (int i = 0; i < 4; ++i) ra4[i] = bload16(ra, aoff, static_cast<uint32_t>(st) * kStage + i * astep);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ss = min(2 * st + j, KS - 1);
      const uint32_t sidx = GK >= 128 ? static_cast<uint32_t>(ss * kSS / group) : static_cast<uint32_t>(ss) * (kSS / GK);
#pragma unroll
      for (int cg = 0; cg < 2; ++cg)
#pragma unroll
        for (int h = 0; h < NS; ++h) snext[j][cg][h] = bload_scale_bits<SD>(rs, soff[cg] + h * sb, sidx * sb);
    }
  };
  // ---- registers -> the wavefront's LDS stage (a wavefront's LDS accesses execute in order: the previous stage's
  // fragment reads are done before these writes land)
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(qs + 1024 * i + ((i & 1) ? qdst1 : qdst0)) = rq4[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(as + 1024 * i + (adst0 ^ (i << 6))) = ra4[i];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int cg = 0; cg < 2; ++cg)
#pragma unroll
        for (int h = 0; h < NS; ++h) scur[j][cg][h] = snext[j][cg][h];
  };
  // ---- compute stage st (the t-th of the wavefront)
  // NSS super-steps (2, or 1 for a last half stage); FAST: the codebook and every scale of the stage are finite in
  // all lanes (uniform), so the tables take the branch-free form and the stage is straight-line code
  auto compute = [&](auto nc, auto fc, int t, int st) {
    constexpr int NSS = decltype(nc)::value;
    constexpr bool FAST = decltype(fc)::value;
#pragma unroll
    for (int j = 0; j < NSS; ++j) {
      const int ss = 2 * st + j;
      const bool rebuild = GK != 256 || (t == 0 && j == 0) || (ss * kSS) % group == 0;  // uniform
      if (rebuild) {
#pragma unroll
        for (int cg = 0; cg < 2; ++cg) {
          const float s = scale_value<SD>(scur[j][cg][0]);
          const bool fast = FAST || (cbw_finite && __builtin_isfinite(s));
          if (GK >= 128) {  // this lane built word g; word w comes from lane group w of the column
            const uint32_t x = lut_word(&cbw[0], s, fast);
#pragma unroll
            for (int w = 0; w < 4; ++w)
              lut[cg][w] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(static_cast<int>(bp0 + 64 * w),
                                                                              static_cast<int>(x)));
          } else if (GK == 64) {  // words 2h, 2h + 1 (h = g & 1); the pair is lane groups g & 2 and (g & 2) + 1
            const uint32_t x0 = lut_word(&cbw[0], s, fast), x1 = lut_word(&cbw[4], s, fast);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              lut[cg][2 * h] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(static_cast<int>(bp0 + 64 * h),
                                                                                  static_cast<int>(x0)));
              lut[cg][2 * h + 1] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(static_cast<int>(bp0 + 64 * h),
                                                                                      static_cast<int>(x1)));
            }
          } else if (kTab) {  // scale bytes are zero-extended u8 loads: & 0xFF only states the table's bound
            const u32x4 t1 = *reinterpret_cast<const u32x4*>(tab + (scur[j][cg][0] & 0xFFu) * 16);
#pragma unroll
            for (int w = 0; w < 4; ++w) lut[cg][w] = t1[w];
            if (GK == 16) {
              const u32x4 t2 = *reinterpret_cast<const u32x4*>(tab + (scur[j][cg][NS - 1] & 0xFFu) * 16);
#pragma unroll
              for (int w = 0; w < 4; ++w) lut2[cg][w] = t2[w];
            }
          } else {
#pragma unroll
            for (int w = 0; w < 4; ++w) lut[cg][w] = lut_word(&cbw[4 * w], s, fast);
            if (GK == 16) {
              const float s2 = scale_value<SD>(scur[j][cg][NS - 1]);
              const bool fast2 = FAST || (cbw_finite && __builtin_isfinite(s2));
#pragma unroll
              for (int w = 0; w < 4; ++w) lut2[cg][w] = lut_word(&cbw[4 * w], s2, fast2);
            }
          }
        }
      }
      v4i af[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
        af[sub] = *reinterpret_cast<const v4i*>(as + c16 * 256 + (((j * 8 + g * 2 + sub) ^ c16) << 4));
#pragma unroll
      for (int cg = 0; cg < 2; ++cg) {
        const int c = cg * 16 + c16;
        const u32x4 pk = *reinterpret_cast<const u32x4*>(qs + c * 128 + (((4 * j + g) ^ ((c >> 1) & 7)) << 4));
        v4i bf[2];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t lo4, hi4;
          if (GK == 16 && w >= 2) lut_decode_word(lut2[cg], pk[w], lo4, hi4);
          else lut_decode_word(lut[cg], pk[w], lo4, hi4);
          bf[w >> 1][(w & 1) * 2] = static_cast<int>(lo4);
          bf[w >> 1][(w & 1) * 2 + 1] = static_cast<int>(hi4);
        }
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) acc[cg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[sub], bf[sub], acc[cg], 0, 0, 0);
      }
    }
  };
  // ---- the next stage loads while this one computes
  if (nst > 0) {
    load(st0);
    store();
  }
  for (int t = 0; t < nst; ++t) {
    if (t + 1 < nst) load(st0 + t + 1);
    {
      const int st = st0 + t;
      bool fin = cbw_finite;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int cg = 0; cg < 2; ++cg)
#pragma unroll
          for (int h = 0; h < NS; ++h) fin = fin && __builtin_isfinite(scale_value<SD>(scur[j][cg][h]));
      const bool all_fin = GK >= 64 && __builtin_amdgcn_ballot_w64(!fin) == 0;  // uniform
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using T = std::true_type;
      using F = std::false_type;
      if (2 * st + 1 < KS) {
        if (GK >= 64 && all_fin) compute(I2{}, T{}, t, st);  // (groups 16 / 32: past 128 VGPRs)
        else compute(I2{}, F{}, t, st);
      } else {
        compute(I1{}, F{}, t, st);
      }
    }
    if (t + 1 < nst) store();
  }

  // ---- the wavefronts' partial sums meet in LDS (the staging area, now free), fixed order
  int32_t* const red = reinterpret_cast<int32_t*>(smem);  // [wave][8 registers][64 lanes]
  __syncthreads();
#pragma unroll
  for (int cg = 0; cg < 2; ++cg)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 8 + cg * 4 + i) * 64 + lane] = acc[cg][i];
  __syncthreads();
  // register rr of lane l: column group rr / 4, row 4 * (l / 16) + rr % 4, column l % 16 (16x16 C layout)
  for (int rr = wave; rr < 8; rr += nw) {
    const int cg = rr >> 2, i = rr & 3;
    const int m = g * 4 + i;
    const int col = static_cast<int>(blockIdx.x) * 32 + cg * 16 + c16;
    if (m >= M || col >= N) continue;
    int a = 0;
    for (int w = 0; w < nw; ++w) a += red[(w * 8 + rr) * 64 + lane];
    const int64_t e = static_cast<int64_t>(m) * N + col;
    if (acc_out) acc_out[e] = a;
    store_out(odt, eager, a, xs[m], sch[col], bias ? load_bias(odt, bias, col) : 0.0f, bias != nullptr, out,
              static_cast<int64_t>(m) * ldo + col);
  }
}

__global__ __launch_bounds__(256) void zero_kernel(u32x4* __restrict__ p, int64_t n16, int32_t* __restrict__ tail,
                                                   int64_t ntail) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n16) p[i] = u32x4{0, 0, 0, 0};
  if (i < ntail) tail[i] = 0;
}

__global__ __launch_bounds__(256) void epilogue_kernel(const int32_t* __restrict__ ws, const float* __restrict__ xs,
                                                       const float* __restrict__ sch, const void* __restrict__ bias,
                                                       int M, int N, void* __restrict__ out, int64_t ldo, int odt,
                                                       bool eager, int32_t* __restrict__ acc_out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<int64_t>(M) * N) return;
  const int m = static_cast<int>(e / N), n = static_cast<int>(e - static_cast<int64_t>(m) * N);
  const int a = ws[e];
  if (acc_out) acc_out[e] = a;
  store_out(odt, eager, a, xs[m], sch[n], bias ? load_bias(odt, bias, n) : 0.0f, bias != nullptr, out,
            static_cast<int64_t>(m) * ldo + n);
}

constexpr int kColTarget = 384;  // workgroups the column kernel aims for (1.5 per CU, 6 wavefronts)

struct Plan {
  int mb, tiles, splits;
  bool col;    // up to 32 rows: gemm_w4_col_kernel (K split over the 4 wavefronts of a workgroup)
  int wsteps;  // col: K-steps per wavefront
};

inline Plan plan(int64_t m, int64_t n, int64_t k) {
  Plan p;
  p.mb = m <= 32 ? 1 : (m <= 64 ? 2 : 4);
  const int kt = static_cast<int>(k / kBK);
  p.col = p.mb == 1;
  if (p.col) {
    p.tiles = static_cast<int>((n + 31) / 32);
    int splits = (kColTarget + p.tiles - 1) / p.tiles;
    const int cap = kt / (4 * kChunk);  // every wavefront keeps at least one chunk
    splits = splits < cap ? splits : cap;
    splits = splits > 1 ? splits : 1;
    p.wsteps = (kt + 4 * splits - 1) / (4 * splits);
    p.splits = (kt + 4 * p.wsteps - 1) / (4 * p.wsteps);
  } else {
    p.tiles = static_cast<int>((n + kBN - 1) / kBN);
    p.splits = (kt + kSteps - 1) / kSteps;
    p.wsteps = 0;
  }
  return p;
}

template <int MB, int SD, int GK>
void launch(const Plan& p, int mode, int odt, const int8_t* a, int64_t lda, const float* xs, const uint8_t* q,
            int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int group, const float* sch,
            const void* bias, int m, int n, int k, void* out, int64_t ldo, int32_t* ws, int32_t* acc_out,
            hipStream_t st) {
  const dim3 grid(p.tiles, p.splits);
  const bool eager = mode == H3K_MODE_EAGER;
  if constexpr (MB == 1) {
    if (p.col && p.splits == 1) {
      hipLaunchKernelGGL((gemm_w4_col_kernel<MB, SD, GK, false>), grid, dim3(256), 0, st, a, lda, xs, q, ldq, s_rel,
                         lds, cb, group, sch, bias, m, n, k, p.wsteps, out, ldo, odt, eager, nullptr, acc_out);
      return;
    }
  }
  if (!p.col && p.splits == 1) {
    hipLaunchKernelGGL((gemm_w4_kernel<MB, SD, GK, false>), grid, dim3(256), 0, st, a, lda, xs, q, ldq, s_rel, lds, cb,
                       group, sch, bias, m, n, k, out, ldo, odt, eager, nullptr, acc_out);
    return;
  }
  const int64_t total = static_cast<int64_t>(m) * n;
  const int64_t n16 = total / 4, ntail = total - n16 * 4;
  const int64_t zt = n16 > ntail ? n16 : ntail;
  hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>((zt + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<u32x4*>(ws), n16, ws + n16 * 4, ntail);
  bool done = false;
  if constexpr (MB == 1) {
    if (p.col) {
      hipLaunchKernelGGL((gemm_w4_col_kernel<MB, SD, GK, true>), grid, dim3(256), 0, st, a, lda, xs, q, ldq, s_rel,
                         lds, cb, group, sch, bias, m, n, k, p.wsteps, out, ldo, odt, eager, ws, acc_out);
      done = true;
    }
  }
  if (!done)
    hipLaunchKernelGGL((gemm_w4_kernel<MB, SD, GK, true>), grid, dim3(256), 0, st, a, lda, xs, q, ldq, s_rel, lds, cb,
                       group, sch, bias, m, n, k, out, ldo, odt, eager, ws, acc_out);
  hipLaunchKernelGGL(epilogue_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, st, ws, xs, sch,
                     bias, m, n, out, ldo, odt, eager, acc_out);
}

// gemm_w4_c16_kernel covers: up to 16 rows, K a multiple of 128, group 16 / 32 / 64 / a multiple of 128, at least
// kC16MinTiles column tiles, and operands whose byte ranges fit a 31-bit buffer offset.  (Two row groups need 158
// VGPRs, one workgroup per CU: 17-32 rows run faster on the 32-row column kernel.)
inline bool c16_ok(int64_t m, int64_t n, int64_t k, int group, int64_t lda, int64_t ldq, int64_t lds, int sbytes) {
  const int64_t lim = (int64_t{1} << 31) - 1;
  return m >= 1 && m <= 16 && k % kSS == 0 && (group == 16 || group == 32 || group == 64 || group % kSS == 0) &&
         (n + 31) / 32 >= kC16MinTiles && (m - 1) * lda + k <= lim && (n - 1) * ldq + k / 2 <= lim &&
         ((n - 1) * lds + k / group) * sbytes <= lim;
}

template <int SD>
void launch_c16(int mode, int odt, const int8_t* a, int64_t lda, const float* xs, const uint8_t* q, int64_t ldq,
                const void* s_rel, int64_t lds, const float* cb, int group, const float* sch, const void* bias, int m,
                int n, int k, void* out, int64_t ldo, int32_t* acc_out, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((n + 31) / 32));
  const int nstg = (k / kSS + 1) / 2;
  const int spw = (nstg + kC16MaxWaves - 1) / kC16MaxWaves;  // stages per wavefront
  const int nw = (nstg + spw - 1) / spw;                       // wavefronts per workgroup, <= kC16MaxWaves
  const bool eager = mode == H3K_MODE_EAGER;
#define H3K_C16(GK)                                                                                                  \
  hipLaunchKernelGGL((gemm_w4_c16_kernel<SD, GK>), grid, dim3(64 * nw), 0, st, a, lda, xs, q, ldq, s_rel, lds, cb,  \
                     group, sch, bias, m, n, k, spw, out, ldo, odt, eager, acc_out)
  if (group == 16) H3K_C16(16);
  else if (group == 32) H3K_C16(32);
  else if (group == 64) H3K_C16(64);
  else if (group == 128) H3K_C16(128);
  else H3K_C16(256);
#undef H3K_C16
}

template <int MB, int SD>
void launch_g(const Plan& p, int mode, int odt, const int8_t* a, int64_t lda, const float* xs, const uint8_t* q,
              int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int group, const float* sch,
              const void* bias, int m, int n, int k, void* out, int64_t ldo, int32_t* ws, int32_t* acc_out,
              hipStream_t st) {
  if (group == 16) launch<MB, SD, 16>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
  else if (group == 32) launch<MB, SD, 32>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
  else launch<MB, SD, 64>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
}

template <int SD>
void launch_m(const Plan& p, int mode, int odt, const int8_t* a, int64_t lda, const float* xs, const uint8_t* q,
              int64_t ldq, const void* s_rel, int64_t lds, const float* cb, int group, const float* sch,
              const void* bias, int m, int n, int k, void* out, int64_t ldo, int32_t* ws, int32_t* acc_out,
              hipStream_t st) {
  if (p.mb == 1) launch_g<1, SD>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
  else if (p.mb == 2) launch_g<2, SD>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
  else launch_g<4, SD>(p, mode, odt, a, lda, xs, q, ldq, s_rel, lds, cb, group, sch, bias, m, n, k, out, ldo, ws, acc_out, st);
}

}  // namespace w4
}  // namespace h3k

using namespace h3k;

extern "C" int64_t h3k_gemm_w4a8_workspace(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % w4::kBK) return 0;
  return w4::plan(m, n, k).splits > 1 ? m * n * static_cast<int64_t>(sizeof(int32_t)) : 0;
}

extern "C" int h3k_gemm_w4a8(const int8_t* a, int64_t lda, const float* xs, const void* q, int64_t ldq,
                             const void* s_rel, int s_dtype, int64_t lds, const float* codebook, int group,
                             const float* s_ch, const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out,
                             int out_dtype, int64_t ldo, int32_t* workspace, int32_t* acc_out, void* stream) {
  if (m < 0 || n < 0 || k < 0 || m > w4::kMaxM || n > (1 << 30) || k > (1 << 17))
    return fail(H3K_EINVAL, "h3k_gemm_w4a8 takes 0..%d rows, got m=%lld n=%lld k=%lld", w4::kMaxM, (long long)m,
                (long long)n, (long long)k);
  if (k % w4::kBK) return fail(H3K_EINVAL, "k=%lld must be a multiple of 64", (long long)k);
  if (!(group == 16 || group == 32 || (group % 64 == 0 && group > 0)) || k % group)
    return fail(H3K_EINVAL, "group_size=%d must be 16, 32 or a multiple of 64 dividing K=%lld", group, (long long)k);
  if (s_dtype != H3K_FP8E4M3 && s_dtype != H3K_F16 && s_dtype != H3K_BF16 && s_dtype != H3K_F32)
    return fail(H3K_EINVAL, "s_rel dtype code %d unsupported (fp8e4m3/f16/bf16/f32)", s_dtype);
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (out_dtype != H3K_BF16 && out_dtype != H3K_F16 && out_dtype != H3K_F32)
    return fail(H3K_EINVAL, "out dtype code %d unsupported", out_dtype);
  if (lda < k || ldq < k / 2 || lds < k / group || ldo < n) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (m == 0 || n == 0) return H3K_OK;
  if (!a || !xs || !q || !s_rel || !codebook || !s_ch || !out) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(a, 16) || lda % 16 || !aligned(q, 16) || ldq % 16)
    return fail(H3K_EINVAL, "a and q must be 16-byte aligned with 16-byte multiple row strides");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mm = static_cast<int>(m), nn = static_cast<int>(n), kk = static_cast<int>(k);
  const uint8_t* qb = static_cast<const uint8_t*>(q);
  const int sbytes = s_dtype == H3K_FP8E4M3 ? 1 : (s_dtype == H3K_F32 ? 4 : 2);
  if (w4::c16_ok(m, n, k, group, lda, ldq, lds, sbytes)) {  // no workspace: K splits inside the workgroup
#define H3K_C(SD) w4::launch_c16<SD>(mode, out_dtype, a, lda, xs, qb, ldq, s_rel, lds, codebook, group, s_ch, bias, \
                                     mm, nn, kk, out, ldo, acc_out, st)
    switch (s_dtype) {
      case H3K_FP8E4M3: H3K_C(H3K_FP8E4M3); break;
      case H3K_F16: H3K_C(H3K_F16); break;
      case H3K_BF16: H3K_C(H3K_BF16); break;
      default: H3K_C(H3K_F32); break;
    }
#undef H3K_C
    return check_launch("gemm_w4a8(c16)");
  }
  const w4::Plan p = w4::plan(m, n, k);
  if (p.splits > 1 && (!workspace || !aligned(workspace, 16)))
    return fail(H3K_EINVAL, "this shape splits K: pass a 16-byte aligned int32 workspace of "
                "h3k_gemm_w4a8_workspace(m, n, k) bytes");
#define H3K_M(SD) w4::launch_m<SD>(p, mode, out_dtype, a, lda, xs, qb, ldq, s_rel, lds, codebook, group, s_ch, bias, \
                                   mm, nn, kk, out, ldo, workspace, acc_out, st)
  switch (s_dtype) {
    case H3K_FP8E4M3: H3K_M(H3K_FP8E4M3); break;
    case H3K_F16: H3K_M(H3K_F16); break;
    case H3K_BF16: H3K_M(H3K_BF16); break;
    default: H3K_M(H3K_F32); break;
  }
#undef H3K_M
  return check_launch("gemm_w4a8");
}
