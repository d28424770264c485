// int8 x int8 -> int32 GEMM on CDNA4 int8 MFMA (v_mfma_i32_32x32x32_i8) with the W4A8 epilogue fused.
//
//   acc[m, n] = sum_k a[m, k] * w8[n, k]                         exact int32 (|acc| < 2^31 for k < 130k)
//   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])          reference h3turbo/h3/qlinear.py:401
//   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))          reference h3turbo/h3/qlinear.py:403
//   bias : out = round(f32(out) + f32(bias[n]))                  reference h3turbo/h3/qlinear.py:404-405
//
// Tiling: a 256-thread workgroup (2 x 2 wavefronts) owns a BM x BN output tile; each wavefront owns
// (BM/2) x (BN/2) as WMB x WNB MFMA 32x32 blocks held in accumulation registers.  K advances 64 bytes per
// step through double-buffered LDS tiles (row-major, 64 B per row, 16-byte chunks XOR-swizzled by row so both
// the 16-byte global->LDS stores and the 16-byte MFMA fragment reads are bank-conflict free).  Operands that
// fall outside M, N or K load as zeros; stores are masked.  Workgroup ids are remapped so each XCD works
// through a contiguous, row-grouped range of tiles (its own L2 then serves the shared A/B panels).
#include "h3k_gemm_common.hpp"

namespace h3k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kGroupM = 8;

__device__ __forceinline__ int swz(int r, int c) { return r * kBK + ((c ^ ((r >> 1) & 3)) << 4); }

// tile id -> (tile_m, tile_n): XCD-contiguous ranges, then groups of kGroupM tile-rows walked column by column
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int xcd = bid & 7, local = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  const int id = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int in_group = kGroupM * tiles_n;
  const int gid = id / in_group;
  const int first_m = gid * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int r = id - gid * in_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

template <int WMB, int WNB, int ODT, bool EAGER>
__global__ __launch_bounds__(256, 1) void gemm_a8w8_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                           const int8_t* __restrict__ B, int64_t ldb, int M, int N, int K,
                                                           const float* __restrict__ xs, const float* __restrict__ sch,
                                                           const void* __restrict__ bias, void* __restrict__ out,
                                                           int64_t ldo, int32_t* __restrict__ acc_out) {
  constexpr int BM = 64 * WMB, BN = 64 * WNB;
  constexpr int A_LD = BM / 64, B_LD = BN / 64;  // 16-byte chunks per thread per K step
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * kBK];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * kBK];

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  uint4 ra[A_LD], rb[B_LD];
  auto gload = [&](int kt) {
    const int kb = kt * kBK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i, r = id >> 2, c = id & 3;
      const int gr = m0 + r, kk = kb + c * 16;
      ra[i] = (gr < M && kk < K) ? *reinterpret_cast<const uint4*>(A + static_cast<int64_t>(gr) * lda + kk)
                                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = tid + 256 * i, r = id >> 2, c = id & 3;
      const int gr = n0 + r, kk = kb + c * 16;
      rb[i] = (gr < N && kk < K) ? *reinterpret_cast<const uint4*>(B + static_cast<int64_t>(gr) * ldb + kk)
                                 : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i, r = id >> 2, c = id & 3;
      *reinterpret_cast<uint4*>(&sA[buf][swz(r, c)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = tid + 256 * i, r = id >> 2, c = id & 3;
      *reinterpret_cast<uint4*>(&sB[buf][swz(r, c)]) = rb[i];
    }
  };

  v16i acc[WMB][WNB];
  static_for<WMB>([&](auto i) { static_for<WNB>([&](auto j) { acc[i][j] = v16i{}; }); });

  const int KT = (K + kBK - 1) / kBK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int arow = wm * (32 * WMB) + (lane & 31), brow = wn * (32 * WNB) + (lane & 31), kh = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    static_for<2>([&](auto s) {
      v4i af[WMB], bf[WNB];
      const int c = s * 2 + kh;
      static_for<WMB>([&](auto i) { af[i] = *reinterpret_cast<const v4i*>(&sA[cur][swz(arow + i * 32, c)]); });
      static_for<WNB>([&](auto j) { bf[j] = *reinterpret_cast<const v4i*>(&sB[cur][swz(brow + j * 32, c)]); });
      static_for<WMB>([&](auto i) {
        static_for<WNB>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        });
      });
    });
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  // C layout of a 32x32 MFMA block: lane l holds column (l % 32); register r holds row
  // (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  static_for<WNB>([&](auto j) {
    const int gn = n0 + wn * (32 * WNB) + j * 32 + (lane & 31);
    const bool nok = gn < N;
    const float sc = nok ? sch[gn] : 0.0f;
    float bv = 0.0f;
    if (bias && nok) {
      if (ODT == H3K_F32) bv = static_cast<const float*>(bias)[gn];
      else if (ODT == H3K_F16) bv = f16_to_f32(static_cast<const uint16_t*>(bias)[gn]);
      else bv = bf16_to_f32(static_cast<const uint16_t*>(bias)[gn]);
    }
    static_for<WMB>([&](auto i) {
      static_for<16>([&](auto r) {
        const int gm = m0 + wm * (32 * WMB) + i * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
        const int a = acc[i][j][decltype(r)::value];
        if (nok && gm < M) {
          if (acc_out) acc_out[static_cast<int64_t>(gm) * N + gn] = a;
          const float xv = xs[gm];
          float f = fp32_round_point(EAGER ? static_cast<float>(a) * fp32_round_point(xv * sc)
                                           : fp32_round_point(static_cast<float>(a) * xv) * sc);
          const int64_t o = static_cast<int64_t>(gm) * ldo + gn;
          if (ODT == H3K_F32) {
            if (bias) f = f + bv;
            static_cast<float*>(out)[o] = f;
          } else if (ODT == H3K_F16) {
            f = round_f16(f);
            if (bias) f = fp32_round_point(f + bv);
            static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_f16_bits(f));
          } else {
            f = round_bf16(f);
            if (bias) f = fp32_round_point(f + bv);
            static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_bf16_bits(f));
          }
        }
      });
    });
  });
}

void gemm_pipe_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                      const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo,
                      int32_t* acc_out, hipStream_t st);
void gemm_persist_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                         const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo,
                         int32_t* acc_out, hipStream_t st);
int gemm_persist_min_k();
void gemm_pipe_mid_launch(int cfg, const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw,
                          const float* s_ch, const void* bias, int m, int n, int k, int mode, void* out, int odt,
                          int64_t ldo, int32_t* acc_out, hipStream_t st);
int cu_count();


// Tile shape of the mid-size pipeline launch: the largest tile that still gives at least 9/16 of the CUs a tile
// (the 128 x 128 tile split over two K groups when its tiles fit in one round: +4-14 % at M = 256-512).
// Measured at M = 64-512, K = 5120 / 13824, N = 5120-15360: 120 tiles of a shape lose to 240 of the next smaller
// one, 160 win against 320.
static int mid_tile(int m, int n) {
  const int enough = cu_count() * 9 / 16;
  auto tiles = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
  if (tiles(128, 256) >= enough) return H3K_MID_128x256;
  // 128 x 128 tiles that all fit in one round run with two K groups: two wavefronts per SIMD instead of one
  if (tiles(128, 128) >= enough) return tiles(128, 128) <= cu_count() ? H3K_MID_128x128_K2 : H3K_MID_128x128;
  if (tiles(64, 128) >= enough) return H3K_MID_64x128;
  return H3K_MID_64x64;
}

template <int WMB, int WNB, int ODT, bool EAGER>
static void launch_gemm(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k, const float* xs,
                        const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc, hipStream_t st) {
  constexpr int BM = 64 * WMB, BN = 64 * WNB;
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_a8w8_kernel<WMB, WNB, ODT, EAGER>), dim3(tiles), dim3(256), 0, st, a, lda, b, ldb, m, n, k, xs,
                     sch, bias, out, ldo, acc);
}

template <int WMB, int WNB>
static void launch_gemm_dt(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int m, int n, int k,
                           const float* xs, const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc,
                           int mode, int odt, hipStream_t st) {
  const bool e = mode == H3K_MODE_EAGER;
#define H3K_L(D, E) launch_gemm<WMB, WNB, D, E>(a, lda, b, ldb, m, n, k, xs, sch, bias, out, ldo, acc, st)
  if (odt == H3K_BF16) { if (e) H3K_L(H3K_BF16, true); else H3K_L(H3K_BF16, false); }
  else if (odt == H3K_F16) { if (e) H3K_L(H3K_F16, true); else H3K_L(H3K_F16, false); }
  else { if (e) H3K_L(H3K_F32, true); else H3K_L(H3K_F32, false); }
#undef H3K_L
}

int gemm_a8w8_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                     const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype, int64_t ldo,
                     int32_t* acc_out, hipStream_t st) {
  if (m < 0 || n < 0 || k < 0 || m > (1 << 30) || n > (1 << 30) || k > (1 << 17))
    return fail(H3K_EINVAL, "bad GEMM shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (k % 16) return fail(H3K_EINVAL, "k=%lld must be a multiple of 16", (long long)k);
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (out_dtype != H3K_BF16 && out_dtype != H3K_F16 && out_dtype != H3K_F32)
    return fail(H3K_EINVAL, "out dtype code %d unsupported", out_dtype);
  if (lda < k || ldw < k || ldo < n) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if (m == 0 || n == 0) return H3K_OK;
  if (!a || !xs || !w8 || !s_ch || !out) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(a, 16) || lda % 16 || !aligned(w8, 16) || ldw % 16)
    return fail(H3K_EINVAL, "int8 operands must be 16-byte aligned with 16-byte multiple row strides");
  const int mm = static_cast<int>(m), nn = static_cast<int>(n), kk = static_cast<int>(k);
  // 256 x 256 tiles once at least 5/8 of the CUs get one and their last round of tiles is not mostly idle; smaller
  // tiles of the same pipeline otherwise.  Measured (K = 5120 / 13824, N = 5120-15360): 160-240 such tiles beat
  // the smaller ones by 10-20 %, 60-80 lose by 2x; at full occupancy 128 x 256 tiles run at 0.83 of the 256 x 256
  // rate, so M=4096 N=5120 (320 tiles: 1.25 rounds) goes faster on 640 tiles of 128 x 256 (+5-14 %).
  const int cus = cu_count();
  const int tiles256 = ((mm + 255) / 256) * ((nn + 255) / 256), tiles128x256 = ((mm + 127) / 128) * ((nn + 255) / 256);
  auto fill = [cus](int t) { return static_cast<double>(t) / (static_cast<double>((t + cus - 1) / cus) * cus); };
  const bool big = k % 64 == 0 && m > 512 && n >= 256 && tiles256 >= cus * 5 / 8 &&
                   fill(tiles256) >= 0.83 * fill(tiles128x256);
  if (big && n % 4 == 0 && k >= gemm_persist_min_k() && aligned(s_ch, 16) && aligned(xs, 16) &&
      (bias == nullptr || aligned(bias, 16)))
    gemm_persist_launch(a, lda, xs, w8, ldw, s_ch, bias, mm, nn, kk, mode, out, out_dtype, ldo, acc_out, st);
  else if (big)
    gemm_pipe_launch(a, lda, xs, w8, ldw, s_ch, bias, mm, nn, kk, mode, out, out_dtype, ldo, acc_out, st);
  else if (k % 64 == 0)
    gemm_pipe_mid_launch(mid_tile(mm, nn), a, lda, xs, w8, ldw, s_ch, bias, mm, nn, kk, mode, out, out_dtype, ldo,
                         acc_out, st);
  else if (m >= 2048 && n >= 256)
    launch_gemm_dt<4, 4>(a, lda, w8, ldw, mm, nn, kk, xs, s_ch, bias, out, ldo, acc_out, mode, out_dtype, st);
  else if (((m + 127) / 128) * ((n + 127) / 128) >= 256)
    launch_gemm_dt<2, 2>(a, lda, w8, ldw, mm, nn, kk, xs, s_ch, bias, out, ldo, acc_out, mode, out_dtype, st);
  else  // fewer 128 x 128 tiles than CUs: 64 x 64 tiles (M=512: N=5120 451 -> 630 TOPS, K=13824 559 -> 738)
    launch_gemm_dt<1, 1>(a, lda, w8, ldw, mm, nn, kk, xs, s_ch, bias, out, ldo, acc_out, mode, out_dtype, st);
  return check_launch("gemm_a8w8");
}

}  // namespace h3k

extern "C" int h3k_gemm_a8w8(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw,
                             const float* s_ch, const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out,
                             int out_dtype, int64_t ldo, int32_t* acc_out, void* stream) {
  return h3k::gemm_a8w8_launch(a, lda, xs, w8, ldw, s_ch, bias, m, n, k, mode, out, out_dtype, ldo, acc_out,
                               static_cast<hipStream_t>(stream));
}
