// Building blocks shared by the int8 MFMA GEMM kernels: wait counters, the LDS barrier, the LDS swizzle and the
// XCD-aware tile order.
#pragma once

#include "h3k_common.hpp"

namespace h3k {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBK = 64;

}  // namespace gemm

// Tile shapes of the mid-size pipeline launch (gemm_pipe_mid_launch)
enum { H3K_MID_64x64 = 0, H3K_MID_64x128 = 1, H3K_MID_128x128 = 2, H3K_MID_128x256 = 3, H3K_MID_128x128_K2 = 4 };

namespace gemm {

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0]+[15:14], expcnt [6:4], lgkmcnt [11:8])
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// Workgroup barrier that orders LDS accesses (and the direct-to-LDS loads the caller has waited for) without
// the memory-model fence of __syncthreads.  The empty asm statements keep the compiler from moving memory
// operations across it; sched_barrier keeps the machine scheduler from doing so.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Tile-rows per group of the XCD-aware tile order (4 and 16 measured no better).
constexpr int kTileGroupRows = 8;

// physical 16-byte chunk of logical chunk c in LDS row r (64-byte rows).  A fragment read takes one chunk of rows
// r0 .. r0 + 31 per half-wavefront; XOR with (r >> 2) & 3 puts every phase of that ds_read_b128 on distinct banks.
// The (r >> 1) ^ (r >> 3) form cost ~4 conflict cycles per read, about 1 % of the GEMMs' time.
__device__ __forceinline__ int swz_chunk(int r, int c) { return c ^ ((r >> 2) & 3); }
__device__ __forceinline__ int swz(int r, int c) { return r * kBK + (swz_chunk(r, c) << 4); }

// tile id -> (tile_m, tile_n): XCD-contiguous ranges, then groups of GM tile-rows walked column by column
template <int GM>
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int xcd = bid & 7, local = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  const int id = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int in_group = GM * tiles_n;
  const int gid = id / in_group;
  const int first_m = gid * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int r = id - gid * in_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

}  // namespace gemm
}  // namespace h3k
