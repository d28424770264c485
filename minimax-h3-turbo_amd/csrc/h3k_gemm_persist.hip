// Persistent large-shape int8 GEMM for gfx950 with the W4A8 epilogue fused (same contract as gemm_pipe_kernel):
//   acc[m, n] = sum_k a[m, k] * w8[n, k]                         exact int32
//   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])          reference h3turbo/h3/qlinear.py:401
//   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))          reference h3turbo/h3/qlinear.py:403
//   bias : out = round(f32(out) + f32(bias[n]))                  reference h3turbo/h3/qlinear.py:404-405
//
// One workgroup per CU (8 wavefronts as 2 x 4, each 128 x 64 outputs = 4 x 2 blocks of v_mfma_i32_32x32x32_i8)
// walks its share of the 256 x 256 output tiles: tile t = blockIdx.x + i * gridDim.x, in the XCD-aware order of
// tile_coords, so each XCD's L2 serves a compact set of operand panels.  K advances 64 bytes per step through an
// S-stage LDS ring filled by direct-to-LDS loads.  The load stream runs straight across tile boundaries: the last
// S steps of a tile issue the next tile's first S stages, which land while the epilogue stores.
//
// The K loop body is the same for every step; the few decisions that change with the step (where the load stream
// points, how many memory ops may stay in flight) are uniform scalar branches, and the per-tile work (pointing the
// load stream at the next tile, fetching its scale vectors) sits behind one of them.
//
// Epilogue.  16-bit outputs leave through a small per-wavefront LDS staging area: each 16-row chunk of the
// wavefront's 128 x 64 block is written in the accumulator layout and read back row-contiguous, so every store
// instruction writes whole 128-byte lines (8 rows x 128 B), non-temporally.  Partial-line stores of a tile make
// the L2 write-allocate and later merge them, and all CUs finish their tiles at nearly the same time; whole-line
// streaming stores take that burst off the L2 and off the loads queued behind it (2.13 -> 1.81 ms for the
// M=32768 K=5120 N=13824 bf16 case at full clock).  fp32 outputs are stored straight from the accumulators.
// Tiles cut by M or N, bias, an accumulator dump or unaligned outputs take the general predicated path.
//
// Wait accounting.  Direct-to-LDS loads and the epilogue's stores count in vmcnt, which retires in issue order.
// Before the barrier of a step, the next stage must have landed; the ops issued after it are normally the S-2
// newer stages (DPW loads each).  In the S-1 steps that follow an epilogue its stores sit in between, so the
// allowance grows by their exact count -- only on the full-tile paths, whose store count is a compile-time
// constant; the general path drains vmcnt itself.  The scale loads of waves 0 and 1 only ever make a wave's
// waits stricter.  The last S steps of a workgroup's last tile wait for everything.
#include "h3k_gemm_common.hpp"

namespace h3k {
namespace persist {

using namespace gemm;

template <int S, int ODT, bool EAGER>
__global__ __launch_bounds__(512, 1) void gemm_persist_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                             const int8_t* __restrict__ B, int64_t ldb, int M, int N,
                                                             int K, const float* __restrict__ xs,
                                                             const float* __restrict__ sch,
                                                             const void* __restrict__ bias, void* __restrict__ out,
                                                             int64_t ldo, int32_t* __restrict__ acc_out, bool vec_out) {
  constexpr int WN = 4, WMB = 4, WNB = 2;  // 2 x 4 wavefronts, 4 x 2 MFMA blocks each
  constexpr int BM = 256, BN = 256;
  constexpr int STAGE = (BM + BN) * kBK;  // 32 KiB per K-step
  constexpr int DPW = STAGE / 1024 / 8;   // 1 KiB direct-to-LDS loads per wavefront per stage
  constexpr bool STAGED = ODT != H3K_F32;
  constexpr int NEPI = STAGED ? 16 : WMB * WNB * 4;  // vector stores of one full-tile epilogue per wavefront
  constexpr int SROW = 144;                          // staging row pitch: 128 bytes of outputs + 16 of padding
  // Scale slots: tile t's xs / s_ch vectors go to slot t % 2.  They are fetched S steps before tile t-1 ends,
  // after tile t-2's epilogue (the last reader of that slot) and the barriers of tile t-1's steps.
  constexpr int RS = 2;
  constexpr int STEADY = DPW * (S - 2);
  static_assert(STEADY + NEPI < 64, "vmcnt allowance out of range");
  // the stage ring, the scale slots (xs[256], s_ch[256] floats each), 8 staging areas of 16 rows
  __shared__ __attribute__((aligned(1024))) int8_t smem[S * STAGE + RS * 2048 + 8 * 16 * SROW];
  float* const sscale = reinterpret_cast<float*>(smem + S * STAGE);

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int T = (tiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  const int KT = K / kBK;  // >= 2 * S (host)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int kh = lane >> 5;

  auto coords = [&](int it, int& m0, int& n0) {
    int tm, tn;
    tile_coords<kTileGroupRows>(static_cast<int>(blockIdx.x) + it * static_cast<int>(gridDim.x), tiles_m, tiles_n, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
  };

  // ---------------------------------------------------------------- load stream
  const int8_t* src[DPW];  // this lane's next 16-byte chunk of each of its DPW rows (rows past M or N repeat the last)
  auto point_loads = [&](int it) {
    int m0, n0;
    coords(it, m0, n0);
    static_for<DPW>([&](auto i) {
      const int d = wave * DPW + i;
      const int lr = lane >> 2;
      if (d < BM / 16) {
        const int r = d * 16 + lr;
        src[i] = A + static_cast<int64_t>(min(m0 + r, M - 1)) * lda + swz_chunk(r, lane & 3) * 16;
      } else {
        const int r = (d - BM / 16) * 16 + lr;
        src[i] = B + static_cast<int64_t>(min(n0 + r, N - 1)) * ldb + swz_chunk(BM + r, lane & 3) * 16;
      }
    });
  };
  // waves 0 and 1: tile it's 256 xs / 256 s_ch values (one 1 KiB direct-to-LDS load each) into scale slot it % RS
  auto load_scales = [&](int it) {
    if (wave < 2) {
      int m0, n0;
      coords(it, m0, n0);
      const float* p = wave == 0 ? xs + (min(m0 + 4 * lane, M - 4) & ~3) : sch + min(n0 + 4 * lane, N - 4);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(p), (lds_void*)(sscale + (it % RS) * 512 + wave * 256),
                                       16, 0, 0);
    }
  };
  auto issue = [&](int buf) {
    int8_t* dst = smem + buf * STAGE + wave * DPW * 1024;
    static_for<DPW>([&](auto i) {
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src[i]), (lds_void*)(dst + i * 1024), 16, 0, 0);
      src[i] += kBK;
    });
  };

  // ---------------------------------------------------------------- fragments and MFMA
  const int arow = wm * (32 * WMB) + (lane & 31), brow = BM + wn * (32 * WNB) + (lane & 31);
  auto read_frags = [&](int buf, int half, v4i (&af)[WMB], v4i (&bf)[WNB]) {
    const int8_t* base = smem + buf * STAGE;
    const int c = half * 2 + kh;
    static_for<WMB>([&](auto i) { af[i] = *reinterpret_cast<const v4i*>(base + swz(arow + i * 32, c)); });
    static_for<WNB>([&](auto j) { bf[j] = *reinterpret_cast<const v4i*>(base + swz(brow + j * 32, c)); });
  };
  v16i acc[WMB][WNB];
  auto zero_acc = [&]() { static_for<WMB>([&](auto i) { static_for<WNB>([&](auto j) { acc[i][j] = v16i{}; }); }); };
  auto mfma = [&](const v4i (&af)[WMB], const v4i (&bf)[WNB]) {
    static_for<WMB>([&](auto i) {
      static_for<WNB>([&](auto j) {
        // operands swapped (B A^T): each lane's accumulators then hold one output row (see the epilogue)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
      });
    });
  };

  // ---------------------------------------------------------------- epilogue
  // Lane l owns output row m = row0 + i * 32 (i < WMB) and, per j < WNB, columns col0 + j * 32 + g * 8 + e
  // (g, e < 4); its scales come from the tile's LDS scale slot.
  int cm0 = 0, cn0 = 0;
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  auto scaled = [&](int a, float x, float s) -> float {
    return fp32_round_point(EAGER ? static_cast<float>(a) * fp32_round_point(x * s)
                                  : fp32_round_point(static_cast<float>(a) * x) * s);
  };
  auto value = [&](int a, float x, float s, float b) -> float {
    float f = scaled(a, x, s);
    if (ODT == H3K_F32) return bias ? f + b : f;
    f = ODT == H3K_F16 ? round_f16(f) : round_bf16(f);
    return bias ? fp32_round_point(f + b) : f;
  };
  auto bits16 = [&](float f) -> uint32_t { return ODT == H3K_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); };
  auto pack4 = [&](const float (&f)[4]) -> uint2 {  // four 16-bit outputs, round to nearest even
    if (ODT == H3K_BF16) {
      const bf16x2 lo = __builtin_convertvector((f32x2){f[0], f[1]}, bf16x2);
      const bf16x2 hi = __builtin_convertvector((f32x2){f[2], f[3]}, bf16x2);
      return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    }
    return make_uint2(bits16(f[0]) | (bits16(f[1]) << 16), bits16(f[2]) | (bits16(f[3]) << 16));
  };
  auto comp = [](const float4& v, int e) { return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w)); };

  // Stores the finished tile.  Returns whether exactly NEPI vector-memory ops were issued (a full-tile path).
  auto epilogue = [&](int slot) -> bool {
    const int row0 = cm0 + wm * (32 * WMB) + (lane & 31);
    const int col0 = cn0 + wn * (32 * WNB) + kh * 4;
    const float* const sx = sscale + slot * 512;
    const bool full = cm0 + BM <= M && cn0 + BN <= N && vec_out && acc_out == nullptr && bias == nullptr;
    const bool lines = (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (ldo & 7) == 0;
    if (full && STAGED && lines) {
      int8_t* const stg = smem + S * STAGE + RS * 2048 + wave * (16 * SROW);
      static_for<WMB>([&](auto i) {
        const float x = sx[row0 - cm0 + i * 32];
        uint2 pk[WNB][4];
        static_for<WNB>([&](auto j) {
          static_for<4>([&](auto g) {
            // element reads: a 16-byte LDS read here makes the compiler drain vmcnt
            const float* p = sx + 256 + col0 - cn0 + j * 32 + g * 8;
            float f[4];
            static_for<4>([&](auto e) { f[e] = scaled(acc[i][j][g * 4 + e], x, p[e]); });
            pk[j][g] = pack4(f);
          });
        });
        static_for<2>([&](auto h) {  // rows h * 16 .. h * 16 + 15 of the 32-row block i
          if (((lane & 31) >> 4) == h) {
            int8_t* w = stg + (lane & 15) * SROW + kh * 8;
            static_for<WNB>([&](auto j) {
              static_for<4>([&](auto g) { *reinterpret_cast<uint2*>(w + (j * 32 + g * 8) * 2) = pk[j][g]; });
            });
          }
          wave_lds_sync();
          static_for<2>([&](auto q) {
            const int rr = (lane >> 3) + 8 * q;
            const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * SROW + (lane & 7) * 16);
            u32x4* dst = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) +
                                                  static_cast<int64_t>(cm0 + wm * (32 * WMB) + i * 32 + h * 16 + rr) * ldo +
                                                  cn0 + wn * (32 * WNB) + (lane & 7) * 8);
            __builtin_nontemporal_store(v, dst);
          });
          wave_lds_sync();  // the next chunk overwrites the staging area
        });
      });
      return true;
    }
    if (full && !STAGED) {  // fp32: one 16-byte store per 4 outputs, straight from the accumulators
      static_for<WMB>([&](auto i) {
        const float x = sx[row0 - cm0 + i * 32];
        const int64_t orow = static_cast<int64_t>(row0 + i * 32) * ldo + col0;
        static_for<WNB>([&](auto j) {
          static_for<4>([&](auto g) {
            const float* p = sx + 256 + col0 - cn0 + j * 32 + g * 8;
            float f[4];
            static_for<4>([&](auto e) { f[e] = scaled(acc[i][j][g * 4 + e], x, p[e]); });
            *reinterpret_cast<float4*>(static_cast<float*>(out) + orow + j * 32 + g * 8) = make_float4(f[0], f[1], f[2], f[3]);
          });
        });
      });
      return true;
    }
    // general path: the xs slot holds whole 16-byte chunks only where they lie inside [0, M), so a tile cut by M
    // reads xs itself
    float xv[WMB];
    if (cm0 + BM <= M) {
      static_for<WMB>([&](auto i) { xv[i] = sx[row0 - cm0 + i * 32]; });
    } else {
      static_for<WMB>([&](auto i) { xv[i] = xs[min(row0 + i * 32, M - 1)]; });
    }
    static_for<WNB>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n = col0 + j * 32 + g * 8;
        const float* sp = sx + 256 + n - cn0;
        const float4 sv = make_float4(sp[0], sp[1], sp[2], sp[3]);
        float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (bias) {
          static_for<4>([&](auto e) {
            if (n + e < N) {
              if (ODT == H3K_F32) bv[e] = static_cast<const float*>(bias)[n + e];
              else if (ODT == H3K_F16) bv[e] = f16_to_f32(static_cast<const uint16_t*>(bias)[n + e]);
              else bv[e] = bf16_to_f32(static_cast<const uint16_t*>(bias)[n + e]);
            }
          });
        }
        static_for<WMB>([&](auto i) {
          const int m = row0 + i * 32;
          if (m < M) {
            int a[4];
            float f[4];
            static_for<4>([&](auto e) {
              a[e] = acc[i][j][g * 4 + e];
              f[e] = value(a[e], xv[i], comp(sv, e), bv[e]);
            });
            const int64_t o = static_cast<int64_t>(m) * ldo + n;
            if (n + 3 < N && vec_out) {
              if (ODT == H3K_F32) {
                *reinterpret_cast<float4*>(static_cast<float*>(out) + o) = make_float4(f[0], f[1], f[2], f[3]);
              } else {
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + o) =
                    make_uint2(bits16(f[0]) | (bits16(f[1]) << 16), bits16(f[2]) | (bits16(f[3]) << 16));
              }
            } else {
              static_for<4>([&](auto e) {
                if (n + e < N) {
                  if (ODT == H3K_F32) static_cast<float*>(out)[o + e] = f[e];
                  else static_cast<uint16_t*>(out)[o + e] = static_cast<uint16_t>(bits16(f[e]));
                }
              });
            }
            if (acc_out) {
              static_for<4>([&](auto e) {
                if (n + e < N) acc_out[static_cast<int64_t>(m) * N + n + e] = a[e];
              });
            }
          }
        });
      });
    });
    // retire this path's own memory ops here, so nothing of unknown count is pending in the next tile's first
    // steps (the compiler would otherwise drain vmcnt at the top of every K-step)
    wait_vmcnt<0>();
    return false;
  };

  // ---------------------------------------------------------------- prologue
  point_loads(0);
  load_scales(0);
  static_for<S>([&](auto s) { issue(s); });
  wait_vmcnt<DPW * (S - 1)>();
  lds_barrier();
  zero_acc();

  v4i a0[WMB], b0[WNB], a1[WMB], b1[WNB];
  read_frags(0, 0, a0, b0);
  int buf = 0;
  bool exact = false;  // the last epilogue issued exactly NEPI vector-memory ops
  for (int it = 0; it < T; ++it) {
    coords(it, cm0, cn0);
    const bool has_next = it + 1 < T;
    for (int kt = 0; kt < KT; ++kt) {
      const bool last = kt == KT - 1;
      if (kt == KT - S && has_next) {  // the load stream moves on to the next tile
        point_loads(it + 1);
        load_scales(it + 1);
      }
      const int nbuf = buf + 1 == S ? 0 : buf + 1;
      read_frags(buf, 1, a1, b1);
      mfma(a0, b0);
      if (!last || has_next) {
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        // stage kt+1 must have landed: normally S-2 newer stages may still be in flight; in the S-1 steps after
        // an epilogue its stores sit in between; at the very end fewer newer stages exist
        if (it > 0 && kt < S - 1) {
          if (exact) wait_vmcnt<STEADY + NEPI>();
          else wait_vmcnt<0>();
        } else if (!has_next && kt >= KT - S) {
          wait_vmcnt<0>();
        } else {
          wait_vmcnt<STEADY>();
        }
        lds_barrier();
        if (has_next || kt < KT - S) issue(buf);  // stage kt+S of this tile, or stage kt+S-KT of the next
      }
      if (!last) read_frags(nbuf, 0, a0, b0);
      mfma(a1, b1);
      buf = nbuf;
    }
    exact = epilogue(it % RS);
    zero_acc();
    if (has_next) read_frags(buf, 0, a0, b0);
  }
}

constexpr int kPersistS = 4;  // ring stages (5 measured no better)

template <int ODT, bool EAGER>
static void launch(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k, const float* xs,
                   const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc, int grid, hipStream_t st) {
  const size_t es = ODT == H3K_F32 ? 4 : 2;
  const bool vec_out = aligned(out, 4 * es) && ldo % 4 == 0;
  hipLaunchKernelGGL((gemm_persist_kernel<kPersistS, ODT, EAGER>), dim3(grid), dim3(512), 0, st, a, lda, b, ldb, m, n,
                     k, xs, sch, bias, out, ldo, acc, vec_out);
}

}  // namespace persist

// Number of compute units of the current device (cached per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Smallest K the persistent kernel takes: its per-tile step phases (the S-1 steps after an epilogue, the S steps
// that issue the next tile) must not overlap.
int gemm_persist_min_k() { return 2 * persist::kPersistS * 64; }

// K % 64 == 0, K >= gemm_persist_min_k(), N % 4 == 0, N >= 256, M >= 4; operands 16-byte aligned with 16-byte
// multiple strides, s_ch, xs and bias 16-byte aligned (checked by the caller)
void gemm_persist_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                         const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo,
                         int32_t* acc_out, hipStream_t st) {
  const int tiles = ((m + 255) / 256) * ((n + 255) / 256);
  const int grid = tiles < cu_count() ? tiles : cu_count();
  const bool e = mode == H3K_MODE_EAGER;
#define H3K_L(D, E) persist::launch<D, E>(a, lda, w8, ldw, m, n, k, xs, s_ch, bias, out, ldo, acc_out, grid, st)
  if (odt == H3K_BF16) { if (e) H3K_L(H3K_BF16, true); else H3K_L(H3K_BF16, false); }
  else if (odt == H3K_F16) { if (e) H3K_L(H3K_F16, true); else H3K_L(H3K_F16, false); }
  else { if (e) H3K_L(H3K_F32, true); else H3K_L(H3K_F32, false); }
#undef H3K_L
}

}  // namespace h3k
