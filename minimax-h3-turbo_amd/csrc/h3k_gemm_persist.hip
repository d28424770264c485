// Persistent large-shape int8 GEMM for gfx950 with the W4A8 epilogue fused (same contract as gemm_pipe_kernel):
//   acc[m, n] = sum_k a[m, k] * w8[n, k]                         exact int32
//   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])          reference h3turbo/h3/qlinear.py:401
//   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))          reference h3turbo/h3/qlinear.py:403
//   bias : out = round(f32(out) + f32(bias[n]))                  reference h3turbo/h3/qlinear.py:404-405
//
// One workgroup per CU walks its share of the 256x256 output tiles (tile t = blockIdx.x + i * gridDim.x, in the
// XCD-aware order of tile_coords, so each XCD's L2 still serves a compact set of operand panels).  The direct-to-
// LDS load stream runs straight across tile boundaries: while a tile's last K-steps are multiplied, the ring is
// already being filled with the next tile's first stages, and those loads land while the epilogue converts and
// stores the finished tile.  The per-tile pipeline fill and drain of a one-tile-per-workgroup launch disappear.
//
// The tile's scale vectors (256 xs values, 256 s_ch values) ride along with its first stage as two more 1 KiB
// direct-to-LDS loads into a small ring, so the epilogue reads them from LDS and no scale lives in registers
// across the main loop.
//
// Wait accounting.  Direct-to-LDS loads and the epilogue's stores count in vmcnt, which retires in issue order.
// Before the barrier of step g the stage g+1 must have landed; ops issued after it are normally the S-2 newer
// stages (DPW loads each).  In the S-1 steps that follow an epilogue, the epilogue's stores sit in between, so the
// allowance grows by their exact count -- only when that count is known at compile time (full tile, vector
// stores, no bias, no accumulator dump); otherwise those waits drain vmcnt completely.  A wave's extra ops (the
// scale loads of waves 0 and 1) only ever make its waits stricter.
#include "h3k_gemm_common.hpp"

namespace h3k {
namespace persist {

using namespace gemm;

template <int WM, int WN, int WMB, int WNB, int S, int ODT, bool EAGER>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_persist_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                                      const int8_t* __restrict__ B, int64_t ldb, int M,
                                                                      int N, int K, const float* __restrict__ xs,
                                                                      const float* __restrict__ sch,
                                                                      const void* __restrict__ bias,
                                                                      void* __restrict__ out, int64_t ldo,
                                                                      int32_t* __restrict__ acc_out, bool vec_out) {
  constexpr int NW = WM * WN;
  constexpr int BM = 32 * WMB * WM, BN = 32 * WNB * WN;
  constexpr int STAGE = (BM + BN) * kBK;
  constexpr int D = STAGE / 1024;
  constexpr int DPW = D / NW;
  static_assert(D % NW == 0 && BM % 16 == 0 && BN % 16 == 0 && S >= 3, "tile shape");
  // vector-memory ops of one full-tile epilogue per wavefront: one store per 4 outputs
  constexpr int NEPI = WMB * WNB * 4;
  static_assert(DPW * (S - 2) + NEPI < 64, "vmcnt allowance out of range");
  static_assert(BM == 256 && BN == 256, "one 1 KiB direct-to-LDS load per scale vector");
  // Scale ring of S + 1 slots: the slot of tile T is refilled for tile T + S + 1, whose first stage is issued at
  // K-step (T + S + 1) * KT - S >= (T + 1) * KT + S * KT - S >= (T + 1) * KT, i.e. after the barrier that follows
  // tile T's epilogue in every wavefront.
  constexpr int RS = S + 1;
  // one LDS object: the stage ring, then the scale ring (RS slots of xs[256] and s_ch[256] floats)
  __shared__ __attribute__((aligned(1024))) int8_t smem[S * STAGE + RS * 2048];
  float* const sscale = reinterpret_cast<float*>(smem + S * STAGE);

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int my_tiles = (tiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  const int KT = K / kBK;
  const int total = my_tiles * KT;  // K-steps this workgroup runs, over all its tiles
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int kh = lane >> 5;

  auto coords = [&](int it, int& m0, int& n0) {
    int tm, tn;
    tile_coords<H3K_PIPE_GM>(static_cast<int>(blockIdx.x) + it * static_cast<int>(gridDim.x), tiles_m, tiles_n, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
  };

  // ---------------------------------------------------------------- load stream (runs S stages ahead)
  const int8_t* src[DPW];
  const float* scale_src = nullptr;  // waves 0 and 1: this lane's 16 bytes of the tile's xs / s_ch vector
  int issue_it = 0, issue_kt = 0;
  auto point_loads = [&](int it) {
    int m0, n0;
    coords(it, m0, n0);
    if (wave == 0) scale_src = xs + (min(m0 + 4 * lane, M - 4) & ~3);
    if (wave == 1) scale_src = sch + min(n0 + 4 * lane, N - 4);
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
  auto issue = [&](int buf) {
    if (issue_kt == 0 && wave < 2) {
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(scale_src),
                                       (lds_void*)(sscale + (issue_it % RS) * 512 + wave * 256), 16, 0, 0);
    }
    static_for<DPW>([&](auto i) {
      int8_t* dst = smem + buf * STAGE + (wave * DPW + i) * 1024;
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src[i] + static_cast<int64_t>(issue_kt) * kBK),
                                       (lds_void*)(dst), 16, 0, 0);
    });
    if (++issue_kt == KT) {
      issue_kt = 0;
      if (++issue_it < my_tiles) point_loads(issue_it);
    }
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

  // ---------------------------------------------------------------- the tile being computed
  // Lane l owns output row m = row0 + i * 32 (i < WMB) and, per j < WNB, columns col0 + j * 32 + g * 8 + e
  // (g, e < 4); its scales come from the tile's LDS scale slot.
  int cm0 = 0, cn0 = 0;

  auto value = [&](int a, float x, float s, float b) -> float {
    float f = fp32_round_point(EAGER ? static_cast<float>(a) * fp32_round_point(x * s)
                                     : fp32_round_point(static_cast<float>(a) * x) * s);
    if (ODT == H3K_F32) return bias ? f + b : f;
    f = ODT == H3K_F16 ? round_f16(f) : round_bf16(f);
    return bias ? fp32_round_point(f + b) : f;
  };
  auto bits16 = [&](float f) -> uint32_t { return ODT == H3K_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); };
  auto comp = [](const float4& v, int e) { return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w)); };


  // Stores the finished tile.  Returns whether exactly NEPI vector-memory ops were issued (with the scale loads
  // the caller adds): true on the unpredicated full-tile path.
  auto epilogue = [&](int slot) -> bool {
    const int row0 = cm0 + wm * (32 * WMB) + (lane & 31);
    const int col0 = cn0 + wn * (32 * WNB) + kh * 4;
    const bool full = cm0 + BM <= M && cn0 + BN <= N && vec_out && acc_out == nullptr && bias == nullptr;
    float xv[WMB];
    if (full) {  // unpredicated: exactly WMB * WNB * 4 stores per wavefront; scales from LDS only
      static_for<WMB>([&](auto i) { xv[i] = sscale[slot * 512 + row0 - cm0 + i * 32]; });
      static_for<WNB>([&](auto j) {
        float4 sv[4];
        static_for<4>([&](auto g) {  // element reads: a 16-byte LDS read here makes the compiler drain vmcnt
          const float* p = sscale + slot * 512 + 256 + col0 - cn0 + j * 32 + g * 8;
          sv[g] = make_float4(p[0], p[1], p[2], p[3]);
        });
        static_for<WMB>([&](auto i) {
          const int64_t orow = static_cast<int64_t>(row0 + i * 32) * ldo + col0 + j * 32;
          static_for<4>([&](auto g) {
            float f[4];
            static_for<4>([&](auto e) { f[e] = value(acc[i][j][g * 4 + e], xv[i], comp(sv[g], e), 0.0f); });
            if (ODT == H3K_F32) {
              *reinterpret_cast<float4*>(static_cast<float*>(out) + orow + g * 8) = make_float4(f[0], f[1], f[2], f[3]);
            } else {
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + orow + g * 8) =
                  make_uint2(bits16(f[0]) | (bits16(f[1]) << 16), bits16(f[2]) | (bits16(f[3]) << 16));
            }
          });
        });
      });
      return true;
    }
    // the xs slot holds whole 16-byte chunks only where they lie inside [0, M): a tile cut by M reads xs itself
    if (cm0 + BM <= M) {
      static_for<WMB>([&](auto i) { xv[i] = sscale[slot * 512 + row0 - cm0 + i * 32]; });
    } else {
      static_for<WMB>([&](auto i) { xv[i] = xs[min(row0 + i * 32, M - 1)]; });
    }
    static_for<WNB>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n = col0 + j * 32 + g * 8;
        const float* sp = sscale + slot * 512 + 256 + n - cn0;
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
    // retire this path's own loads here, so the compiler sees nothing pending at the top of the main loop (it
    // would otherwise drain vmcnt there on every K-step); the waits after this epilogue drain it anyway
    wait_vmcnt<0>();
    return false;
  };

  // ---------------------------------------------------------------- prologue
  coords(0, cm0, cn0);
  point_loads(0);
  static_for<S>([&](auto s) {
    if (s < total) issue(s);
  });
  if (total >= S) wait_vmcnt<DPW * (S - 1)>();
  else wait_vmcnt<0>();
  lds_barrier();
  zero_acc();

  v4i a0[WMB], b0[WNB], a1[WMB], b1[WNB];
  read_frags(0, 0, a0, b0);
  int buf = 0, ckt = 0, cit = 0;
  int since_epi = S;      // K-steps since the last epilogue (>= S: outside the window)
  bool epi_exact = false;  // the last epilogue issued exactly NEPI vector-memory ops
  for (int g = 0; g < total; ++g) {
    const int nbuf = buf + 1 == S ? 0 : buf + 1;
    ++since_epi;
    read_frags(buf, 1, a1, b1);
    mfma(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
    // stage g+1 must have landed; stages g+2 .. g+S-1 (and a recent epilogue's ops) may be in flight
    if (g + S <= total) {
      if (since_epi >= S) wait_vmcnt<DPW * (S - 2)>();
      else if (epi_exact) wait_vmcnt<DPW * (S - 2) + NEPI>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if (g + S < total) issue(buf);
    const bool tile_end = ckt + 1 == KT;
    if (!tile_end && g + 1 < total) read_frags(nbuf, 0, a0, b0);
    mfma(a1, b1);
    buf = nbuf;
    if (tile_end) {  // the next stage's fragments are read after the epilogue: fewer registers live across it
      epi_exact = epilogue(cit % RS);
      ckt = 0;
      since_epi = 0;
      zero_acc();
      if (++cit < my_tiles) coords(cit, cm0, cn0);
      if (g + 1 < total) read_frags(nbuf, 0, a0, b0);
    } else {
      ++ckt;
    }
  }
}

#ifndef H3K_PERSIST_S
#define H3K_PERSIST_S 4
#endif


template <int ODT, bool EAGER>
static void launch(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k, const float* xs,
                   const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc, int grid, hipStream_t st) {
  constexpr int WM = 2, WN = 4, WMB = 4, WNB = 2;
  const size_t es = ODT == H3K_F32 ? 4 : 2;
  const bool vec_out = aligned(out, 4 * es) && ldo % 4 == 0;
  hipLaunchKernelGGL((gemm_persist_kernel<WM, WN, WMB, WNB, H3K_PERSIST_S, ODT, EAGER>), dim3(grid), dim3(WM * WN * 64), 0,
                     st, a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, vec_out);
}

}  // namespace persist

// Number of compute units of the current device (cached per device).
static int cu_count() {
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

// K % 64 == 0, N % 4 == 0, N >= 256, M >= 1; operands 16-byte aligned with 16-byte multiple strides, s_ch and
// bias 16-byte aligned (checked by the caller)
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
