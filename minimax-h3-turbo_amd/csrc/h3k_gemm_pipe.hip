// Large-shape int8 x int8 -> int32 GEMM for gfx950 with the W4A8 epilogue fused: the deep-pipeline variant.
//
// Same contract as gemm_a8w8_kernel (h3k_gemm.hip):
//   acc[m, n] = sum_k a[m, k] * w8[n, k]                         exact int32
//   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])          reference h3turbo/h3/qlinear.py:401
//   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))          reference h3turbo/h3/qlinear.py:403
//   bias : out = round(f32(out) + f32(bias[n]))                  reference h3turbo/h3/qlinear.py:404-405
// for K a multiple of 64.
//
// Data movement: global -> LDS with the gfx950 direct-to-LDS load (global_load_lds_dwordx4: each lane's 16
// bytes land at M0 + 16 * lane, no register staging), into a ring of S stages of BK = 64 bytes of K.  Stage
// kt + S is issued as soon as every wave has finished reading stage kt, so S - 1 stages of loads are in flight
// while one is multiplied: the HBM/L2 latency is hidden behind (S - 1) x BM x BN x 64 MACs of MFMA work.
// Waits are explicit (s_waitcnt vmcnt / lgkmcnt, then s_barrier) instead of __syncthreads, whose release fence
// would drain every outstanding load, prefetches included.
//
// LDS layout of a stage: A rows [BM][64 B] then B rows [BN][64 B].  The four 16-byte chunks of a row are
// XOR-swizzled by (row >> 2) & 3, so the 16-byte MFMA fragment reads (32 rows x one chunk per half-wave) are
// bank-conflict free.  A direct-to-LDS load writes 1 KiB contiguously (16 rows); the swizzle is applied on the
// global side instead, by choosing which chunk each lane fetches.  Rows past M or N are clamped to the last
// valid row (their products only reach output rows/columns that are never stored).
//
// MFMA: v_mfma_i32_32x32x32_i8.  The workgroup (KS groups of WM x WN wavefronts) owns a BM x BN output tile; a
// wavefront owns (BM / WM) x (BN / WN) as WMB x WNB blocks of 32 x 32 held in accumulation registers.  With KS > 1
// the groups take turns over the K-steps (group g multiplies the steps kt with kt / U = g mod KS), which puts KS
// wavefronts on each SIMD for a tile that has a CU to itself; at the end each group adds the others' sums of the
// 32-row blocks it stores (exact int32, through LDS) and stores those.  Within a K-step
// the two 32-byte halves are software-pipelined: fragments of half 1 are read while half 0 multiplies, and
// the fragments of the next K-step's half 0 while half 1 multiplies.
#include "h3k_gemm_common.hpp"

namespace h3k {

namespace pipe {

using namespace gemm;

template <int WM, int WN, int WMB, int WNB, int S, int U, int MINB, int ODT, bool EAGER, int KS = 1>
__global__ __launch_bounds__(KS * WM * WN * 64, MINB) void gemm_pipe_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                                    const int8_t* __restrict__ B, int64_t ldb, int M,
                                                                    int N, int K, const float* __restrict__ xs,
                                                                    const float* __restrict__ sch,
                                                                    const void* __restrict__ bias,
                                                                    void* __restrict__ out, int64_t ldo,
                                                                    int32_t* __restrict__ acc_out, bool vec_out,
                                                                    bool vec_acc) {
  constexpr int NT = WM * WN;  // wavefronts per K group
  constexpr int NW = KS * NT;
  constexpr int UP = KS * U;    // stages read between two barriers (U per group)
  constexpr int BM = 32 * WMB * WM, BN = 32 * WNB * WN;
  constexpr int STAGE = (BM + BN) * kBK;           // bytes per stage
  constexpr int D = STAGE / 1024;                  // 1 KiB direct-to-LDS loads per stage
  constexpr int DPW = D / NW;                      // ... per wavefront
  static_assert(D % NW == 0, "stage loads must split evenly over the wavefronts");
  static_assert(BM % 16 == 0 && BN % 16 == 0, "16-row load granules");
  static_assert(U >= 1 && S >= 2 * UP, "a group of UP stages is read while the next UP land");
  static_assert(WMB % KS == 0, "each K group stores WMB / KS of the 32-row blocks");
  static_assert(KS == 1 || NW * (WMB / KS) * WNB * 4096 <= S * STAGE, "the sums handed over fit in the ring");
  __shared__ __attribute__((aligned(1024))) int8_t smem[S * STAGE];

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords<kTileGroupRows>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave / NT, wt = wave % NT;  // K group, wavefront within the group
  const int wm = wt / WN, wn = wt % WN;

  // per-lane global source of each of this wave's DPW loads (K offset added per stage)
  const int8_t* src[DPW];
  static_for<DPW>([&](auto i) {
    const int d = wave * DPW + i;  // load granule within the stage
    const int lr = (lane >> 2);
    if (d < BM / 16) {
      const int r = d * 16 + lr;
      const int c = swz_chunk(r, lane & 3);
      const int gr = min(m0 + r, M - 1);
      src[i] = A + static_cast<int64_t>(gr) * lda + c * 16;
    } else {
      const int r = (d - BM / 16) * 16 + lr;
      const int c = swz_chunk(BM + r, lane & 3);
      const int gr = min(n0 + r, N - 1);
      src[i] = B + static_cast<int64_t>(gr) * ldb + c * 16;
    }
  });
  auto issue = [&](int kt, int buf) {
    static_for<DPW>([&](auto i) {
      int8_t* dst = smem + buf * STAGE + (wave * DPW + i) * 1024;
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src[i] + static_cast<int64_t>(kt) * kBK),
                                       (lds_void*)(dst), 16, 0, 0);
    });
  };

  const int arow = wm * (32 * WMB) + (lane & 31), brow = BM + wn * (32 * WNB) + (lane & 31), kh = lane >> 5;
  auto read_frags = [&](int buf, int half, v4i (&af)[WMB], v4i (&bf)[WNB]) {
    const int8_t* base = smem + buf * STAGE;
    const int c = half * 2 + kh;
    static_for<WMB>([&](auto i) { af[i] = *reinterpret_cast<const v4i*>(base + swz(arow + i * 32, c)); });
    static_for<WNB>([&](auto j) { bf[j] = *reinterpret_cast<const v4i*>(base + swz(brow + j * 32, c)); });
  };

  v16i acc[WMB][WNB];
  static_for<WMB>([&](auto i) { static_for<WNB>([&](auto j) { acc[i][j] = v16i{}; }); });
  auto mfma = [&](const v4i (&af)[WMB], const v4i (&bf)[WNB]) {
    static_for<WMB>([&](auto i) {
      static_for<WNB>([&](auto j) {
        // operands swapped (B A^T): the accumulator layout then gives each lane one output row (see epilogue)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
      });
    });
  };

  const int KT = K / kBK;  // a multiple of UP when KS > 1 (launcher)
  auto ring = [](int b) { return b >= S ? b - S : b; };
  // prologue: fill the ring, wait for the first UP stages
  static_for<S>([&](auto s) {
    if (s < KT) issue(s, s);
  });
  int issued = KT < S ? KT : S;
  if (KT >= S) wait_vmcnt<DPW * (S - UP)>();
  else wait_vmcnt<0>();
  lds_barrier();

  // Groups of UP K-steps between barriers, U of them per K group.  At the barrier closing group kt the next
  // group's stages must have landed; stages issued after them (at most S - 2 UP) may still be in flight.  The UP
  // buffers just read are then refilled with the stages UP steps ahead.
  v4i a0[WMB], b0[WNB], a1[WMB], b1[WNB];
  read_frags(g * U, 0, a0, b0);
  int buf = 0;  // ring buffer of step kt
  for (int kt = 0; kt < KT; kt += UP) {
    static_for<U>([&](auto u) {
      const int sb = ring(buf + g * U + u);  // this group's stage
      read_frags(sb, 1, a1, b1);
      mfma(a0, b0);
      if (u + 1 < U) {
        read_frags(ring(sb + 1), 0, a0, b0);
        mfma(a1, b1);
      } else {
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        if (issued == kt + S && kt + S <= KT) wait_vmcnt<DPW * (S - 2 * UP)>();
        else wait_vmcnt<0>();
        lds_barrier();
        static_for<UP>([&](auto v) {
          if (issued < KT) {
            issue(issued, ring(buf + v));
            ++issued;
          }
        });
        if (kt + UP < KT) read_frags(ring(buf + UP + g * U), 0, a0, b0);
        mfma(a1, b1);
      }
    });
    buf = ring(buf + UP);
  }
  if constexpr (KS > 1) {
    // The loop's last barrier came after every wave's last fragment read and after vmcnt(0): the ring is free.
    // Group h hands the 32-row blocks i with i % KS != h to group i % KS, one 4 KiB slot per block, lane-major.
    constexpr int HB = WMB / KS;  // blocks each group stores
    int32_t* const xch = reinterpret_cast<int32_t*>(smem);
    auto slot = [&](int h, int i, int j) { return xch + (((wt * KS + h) * HB + i / KS) * WNB + j) * 1024 + lane * 4; };
    static_for<WMB>([&](auto i) {
      if (i % KS != g) {
        static_for<WNB>([&](auto j) {
          static_for<4>([&](auto q) {
            *reinterpret_cast<v4i*>(slot(g, i, j) + q * 256) =
                v4i{acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]};
          });
        });
      }
    });
    wait_lgkmcnt0();
    lds_barrier();
    static_for<WMB>([&](auto i) {
      if (i % KS == g) {
        for (int h = 0; h < KS; ++h) {
          if (h == g) continue;
          static_for<WNB>([&](auto j) {
            static_for<4>([&](auto q) {
              const v4i v = *reinterpret_cast<const v4i*>(slot(h, i, j) + q * 256);
              static_for<4>([&](auto e) { acc[i][j][q * 4 + e] += v[static_cast<int>(e)]; });
            });
          });
        }
      }
    });
  }

  // ---------------------------------------------------------------- epilogue
  // With the operands swapped, block (i, j) holds C^T: lane l owns output row m = i * 32 + (l % 32) and
  // register r the column n = j * 32 + (r / 4) * 8 + (l / 32) * 4 + (r % 4), i.e. four consecutive columns per
  // r / 4, stored with one 8-byte (16-bit outputs) or 16-byte (fp32 / int32) store.  Scales are loaded once.
  const int mrow = m0 + wm * (32 * WMB) + (lane & 31);
  const int ncol = n0 + wn * (32 * WNB) + kh * 4;
  float xv[WMB];
  static_for<WMB>([&](auto i) {
    const int m = mrow + i * 32;
    xv[i] = m < M ? xs[m] : 0.0f;
  });
  auto value = [&](int a, float x, float s, float b) -> float {
    float f = fp32_round_point(EAGER ? static_cast<float>(a) * fp32_round_point(x * s)
                                     : fp32_round_point(static_cast<float>(a) * x) * s);
    if (ODT == H3K_F32) return bias ? f + b : f;
    f = ODT == H3K_F16 ? round_f16(f) : round_bf16(f);
    return bias ? fp32_round_point(f + b) : f;
  };
  auto bits16 = [&](float f) -> uint32_t { return ODT == H3K_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); };
  static_for<WNB>([&](auto j) {
    float sc[16], bv[16];
    static_for<16>([&](auto r) {
      const int n = ncol + j * 32 + (r >> 2) * 8 + (r & 3);
      sc[r] = n < N ? sch[n] : 0.0f;
      float b = 0.0f;
      if (bias && n < N) {
        if (ODT == H3K_F32) b = static_cast<const float*>(bias)[n];
        else if (ODT == H3K_F16) b = f16_to_f32(static_cast<const uint16_t*>(bias)[n]);
        else b = bf16_to_f32(static_cast<const uint16_t*>(bias)[n]);
      }
      bv[r] = b;
    });
    static_for<WMB>([&](auto i) {
      const int m = mrow + i * 32;
      if (m < M && (KS == 1 || i % KS == g)) {
        static_for<4>([&](auto q) {
          const int n = ncol + j * 32 + q * 8;
          int a[4];
          float f[4];
          static_for<4>([&](auto e) {
            a[e] = acc[i][j][q * 4 + e];
            f[e] = value(a[e], xv[i], sc[q * 4 + e], bv[q * 4 + e]);
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
            const int64_t oa = static_cast<int64_t>(m) * N + n;
            if (n + 3 < N && vec_acc) {
              *reinterpret_cast<int4*>(acc_out + oa) = make_int4(a[0], a[1], a[2], a[3]);
            } else {
              static_for<4>([&](auto e) {
                if (n + e < N) acc_out[oa + e] = a[e];
              });
            }
          }
        });
      }
    });
  });
}

// The 256 x 256 tile: (WM, WN, WMB, WNB, S stages, U stages per barrier, workgroups per CU).  5 stages and two
// K-steps per barrier measured no better.
constexpr int cWM = 2, cWN = 4, cWMB = 4, cWNB = 2, cS = 4, cU = 1, cMINB = 1;  // 8 waves

template <int ODT, bool EAGER>
static void launch_pipe(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k,
                        const float* xs, const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc,
                        hipStream_t st) {
  constexpr int BM = 32 * cWMB * cWM, BN = 32 * cWNB * cWN;
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  // vector stores of 4 consecutive outputs need their address aligned to 4 elements
  const size_t es = ODT == H3K_F32 ? 4 : 2;
  const bool vec_out = aligned(out, 4 * es) && ldo % 4 == 0;
  const bool vec_acc = acc == nullptr || (aligned(acc, 16) && n % 4 == 0);
  if ((k / kBK) % cU == 0)
    hipLaunchKernelGGL((gemm_pipe_kernel<cWM, cWN, cWMB, cWNB, cS, cU, cMINB, ODT, EAGER>), dim3(tiles),
                       dim3(cWM * cWN * 64), 0, st, a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, vec_out, vec_acc);
  else  // K-step count not a multiple of the group: one stage per barrier
    hipLaunchKernelGGL((gemm_pipe_kernel<cWM, cWN, cWMB, cWNB, 4, 1, cMINB, ODT, EAGER>), dim3(tiles),
                       dim3(cWM * cWN * 64), 0, st, a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, vec_out, vec_acc);
}

// Smaller tiles for shapes with few 256 x 256 tiles (M up to a few thousand rows): the same deep direct-to-LDS
// pipeline, U K-steps per barrier where the K-step count is a multiple of U (one otherwise).  The register-staged
// kernel of h3k_gemm.hip keeps a single K-step in flight and is latency-bound there.
template <int WM, int WN, int WMB, int WNB, int S, int U, int MINB, int ODT, bool EAGER, int KS = 1>
static void launch_mid(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k,
                       const float* xs, const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc,
                       hipStream_t st) {
  constexpr int BM = 32 * WMB * WM, BN = 32 * WNB * WN;
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  const size_t es = ODT == H3K_F32 ? 4 : 2;
  const bool vec_out = aligned(out, 4 * es) && ldo % 4 == 0;
  const bool vec_acc = acc == nullptr || (aligned(acc, 16) && n % 4 == 0);
  if ((U > 1 || KS > 1) && (k / kBK) % (KS * U) == 0)
    hipLaunchKernelGGL((gemm_pipe_kernel<WM, WN, WMB, WNB, S, U, MINB, ODT, EAGER, KS>), dim3(tiles),
                       dim3(KS * WM * WN * 64), 0, st, a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, vec_out,
                       vec_acc);
  else
    hipLaunchKernelGGL((gemm_pipe_kernel<WM, WN, WMB, WNB, S, 1, MINB, ODT, EAGER>), dim3(tiles), dim3(WM * WN * 64), 0,
                       st, a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, vec_out, vec_acc);
}

// Ring depths of the two larger mid-size tiles.  4-6 stages (128 x 256) and 3-5 (128 x 128) measured within run-to-run
// noise of each other at M = 128-1024, K = 5120 / 13824, N = 5120-15360.  Two K-steps per barrier make the 64-row
// tiles faster (64 x 64 +12-14 %, 64 x 128 +2-7 %) and the 128-row ones slower (-7 to -11 %).
constexpr int kMidS128x256 = 5, kMidS128x128 = 4;
// The 128 x 128 tile with two K groups (one round of tiles, one workgroup per CU): 6 stages against 4, 7 and 8, and
// one K-step per group between barriers against two, at M = 256-512 on the four (K, N) pairs: 4 stages lost 2-7 %
// to the single-group tile, 6 gained 4-14 %, two K-steps per group lost 0-6 %.
constexpr int kMidS128x128K2 = 6;


template <int ODT, bool EAGER>
static void launch_mid_cfg(int cfg, const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k,
                           const float* xs, const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc,
                           hipStream_t st) {
  switch (cfg) {
    case H3K_MID_128x256:  // 8 waves of 64 x 64, 5 stages of 24 KiB, one workgroup per CU
      launch_mid<2, 4, 2, 2, kMidS128x256, 1, 1, ODT, EAGER>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, st);
      break;
    case H3K_MID_128x128_K2:  // 2 K groups of 4 waves of 64 x 64, 6 stages of 16 KiB, one workgroup per CU
      launch_mid<2, 2, 2, 2, kMidS128x128K2, 1, 1, ODT, EAGER, 2>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc,
                                                                  st);
      break;
    case H3K_MID_128x128:  // 4 waves of 64 x 64, 4 stages of 16 KiB, two workgroups per CU
      launch_mid<2, 2, 2, 2, kMidS128x128, 1, 2, ODT, EAGER>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, st);
      break;
    case H3K_MID_64x128:  // 4 waves of 32 x 64, 5 stages of 12 KiB, two workgroups per CU, 2 K-steps per barrier
      launch_mid<2, 2, 1, 2, 5, 2, 2, ODT, EAGER>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, st);
      break;
    default:  // 64 x 64: 4 waves of 32 x 32, 8 stages of 8 KiB, two workgroups per CU, 2 K-steps per barrier
      launch_mid<2, 2, 1, 1, 8, 2, 2, ODT, EAGER>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, st);
      break;
  }
}

}  // namespace pipe

// Mid-size launch: K % 64 == 0, operands as for gemm_pipe_launch; cfg is one of the H3K_MID_* tile shapes.
void gemm_pipe_mid_launch(int cfg, const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw,
                          const float* s_ch, const void* bias, int m, int n, int k, int mode, void* out, int odt,
                          int64_t ldo, int32_t* acc_out, hipStream_t st) {
  const bool e = mode == H3K_MODE_EAGER;
#define H3K_L(D, E) pipe::launch_mid_cfg<D, E>(cfg, a, lda, w8, ldw, m, n, k, xs, s_ch, bias, out, ldo, acc_out, st)
  if (odt == H3K_BF16) { if (e) H3K_L(H3K_BF16, true); else H3K_L(H3K_BF16, false); }
  else if (odt == H3K_F16) { if (e) H3K_L(H3K_F16, true); else H3K_L(H3K_F16, false); }
  else { if (e) H3K_L(H3K_F32, true); else H3K_L(H3K_F32, false); }
#undef H3K_L
}

// K % 64 == 0, operands 16-byte aligned with 16-byte multiple strides (checked by the caller)
void gemm_pipe_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                      const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo,
                      int32_t* acc_out, hipStream_t st) {
  const bool e = mode == H3K_MODE_EAGER;
#define H3K_L(D, E) pipe::launch_pipe<D, E>(a, lda, w8, ldw, m, n, k, xs, s_ch, bias, out, ldo, acc_out, st)
  if (odt == H3K_BF16) { if (e) H3K_L(H3K_BF16, true); else H3K_L(H3K_BF16, false); }
  else if (odt == H3K_F16) { if (e) H3K_L(H3K_F16, true); else H3K_L(H3K_F16, false); }
  else { if (e) H3K_L(H3K_F32, true); else H3K_L(H3K_F32, false); }
#undef H3K_L
}

}  // namespace h3k
