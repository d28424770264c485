// Large-shape int8 GEMM over a fragment-ordered ("packed") int8 weight grid, W4A8 epilogue fused:
//   acc[m, n] = sum_k a[m, k] * w8[n, k]                         exact int32
//   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])          reference h3turbo/h3/qlinear.py:401
//   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))          reference h3turbo/h3/qlinear.py:403
//   bias : out = round(f32(out) + f32(bias[n]))                  reference h3turbo/h3/qlinear.py:404-405
//
// Packed weight layout.  The grid is cut into K-steps of 64 bytes and blocks of 32 weight rows, N padded with zero
// rows to a multiple of 256 (a whole output tile).  Step t, block b is 2 KiB at ((t * NBP + b) * 2 + h) * 1024 +
// lane * 16 (NBP = padded N / 32): the 16-byte MFMA fragment of lane `lane` for half h, i.e. row 32b + (lane & 31),
// bytes 64t + 32(lane >> 5) + 16h .. + 16.  Lanes 0-31 own the first 32 bytes of the step, lanes 32-63 the last
// 32; any permutation of k applied to both operands leaves the dot products unchanged, and the activation fragments
// are read from LDS in the same order.  One 16-byte load per lane fetches a whole 1 KiB fragment, and the 4 blocks a
// wavefront multiplies at one step are 8 KiB in one piece.
//
// Why: the row-major kernels stage both operands through LDS, and at full MFMA rate their 96 KiB of fragment reads
// plus 32 KiB of direct-to-LDS writes per K-step (256 x 256 tile) run the LDS at 60-75 % of its measured read
// rate, a co-limiter next to the power ceiling.  Here only the activations go through LDS: a workgroup of 4
// wavefronts (one per SIMD) owns a 256 x 256 tile.  For 16-bit outputs (LAY 1) they split it 1 x 4, each wavefront
// 256 x 64 outputs as 8 x 2 blocks of v_mfma_i32_32x32x32_i8, so no weight fragment is loaded by two wavefronts;
// per K-step the LDS sees 16 KiB of DMA writes and 64 KiB of fragment reads.  fp32 outputs and the accumulator dump
// (LAY 0) split it 2 x 2, 128 x 128 as 4 x 4 blocks (32 KiB of fragment reads, each weight fragment loaded twice).
// The weight fragments go straight from L2 into registers through buffer loads, S K-steps ahead, in a register
// ring of S x 16 VGPRs (LAY 1; S x 32 for LAY 0).
//
// Schedule (the persistent form of h3k_gemm_persist.hip): one workgroup per CU walks tiles t = blockIdx +
// i * gridDim in the XCD-aware order of tile_coords; the activation DMA stream and the weight register stream both
// run across tile boundaries (the last S steps of a tile issue the next tile's first S steps).  Per step, after
// the barrier: the DMA of stage kt + S into the stage just read; after the second half's MFMAs: the weight
// fragments of step kt + S into the registers just consumed.  vmcnt retires in issue order, so the wait before a
// step's barrier allows exactly the ops of the S - 2 newer steps (G each) -- plus, in the S - 1 steps after a
// full-tile epilogue, its NEPI stores.  Each tile's K loop is peeled into its first S steps, the steady steps and
// its last S steps, so that the steady steps carry no branch at all (a taken branch stalls the wave's MFMA
// stream while the instruction buffer refills); the first step's first MFMAs start from a zero accumulator, so
// nothing clears the 256 accumulator registers between tiles.  The instruction order of the whole region between
// two barriers is pinned (sched_group_barrier): each half-step's MFMAs with the other half's fragment reads going
// out one per MFMA.  The 16-bit epilogue stages each 32-row block of a wavefront's raw accumulators through a
// private LDS area (two buffers on whole tiles, the next block staged while this one is read back), reads 8
// consecutive columns of a row per lane (their scales and bias are fixed per lane for the whole tile) and stores
// whole 128-byte lines, non-temporally, with the next tile's loads still in flight.
#include "h3k_gemm_common.hpp"

namespace h3k {
namespace w8p {

using namespace gemm;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

constexpr int kBlockBytes = 2048;  // one 32-row block, one 64-byte K-step

// Buffer descriptor of the packed weights as four scalar words (base, stride 0, num_records, raw-buffer flags).
__device__ __forceinline__ u32x4 weight_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

// One 16-byte weight fragment load into registers, as inline assembly.  The compiler's wait insertion treats the
// direct-to-LDS loads and register-returning buffer loads as counters that may retire out of order, and where both
// are pending it can only wait for vmcnt(0): with builtin loads it drained vmcnt at the top of every group of S
// steps.  The assembly load is invisible to it, and the kernel's explicit waits cover it: the fragments of step kt
// are part of the group whose arrival the wait before step kt - 1's barrier enforces.  Nothing but an MFMA reads
// the destination registers, and none before that wait.
// An fp32 value materialised as such (see fp32_round_point), as a plain asm statement rather than a volatile one:
// it orders nothing else, so the scheduler stays free to overlap the epilogue's LDS reads with its arithmetic.
__device__ __forceinline__ float value_point(float f) {
  __asm__("" : "+v"(f));
  return f;
}

template <int OFF>
__device__ __forceinline__ void weight_load(v4i& dst, const u32x4& rsrc, uint32_t voff, uint32_t soff) {
  __asm__ volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:%4"
                   : "=&v"(dst)
                   : "v"(voff), "s"(rsrc), "s"(soff), "n"(OFF));
}

constexpr int kEarlyMfma = 2;  // MFMAs of a first half-step issued before the second half's fragment reads


// Epilogue variants (a template parameter, so that no per-element branch splits the epilogue's code):
enum { EPI_PLAIN16 = 0, EPI_BIAS16 = 1, EPI_GENERAL = 2, EPI_ACC = 3 };

template <int S, int ODT, bool EAGER, int EPI, int LAY>
__global__ __launch_bounds__(256, 1) void gemm_w8p_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                          const int8_t* __restrict__ Bp, uint32_t bp_bytes, int NBP,
                                                          int M, int N, int K, const float* __restrict__ xs,
                                                          const float* __restrict__ sch, const void* __restrict__ bias,
                                                          void* __restrict__ out, int64_t ldo,
                                                          int32_t* __restrict__ acc_out, bool vec_out, int tiles_dp,
                                                          int P, int KP, int32_t* __restrict__ part) {
  // LAY 0: 2 x 2 wavefronts of 128 x 128 outputs (4 x 4 blocks of 32 x 32); LAY 1: 1 x 4 wavefronts of 256 x 64
  // (8 x 2 blocks), whose weight fragments no two wavefronts share (16-bit epilogues only).
  constexpr int WMB = LAY ? 8 : 4, WNB = LAY ? 2 : 4;
  constexpr int WROWS = 32 * WMB, WCOLS = 32 * WNB;  // a wavefront's output rows and columns
  constexpr int LPR = WCOLS / 8;  // staged read-back: lanes per output row (8 columns each)
  constexpr int RPR = 64 / LPR;   // ... rows per read-back instruction
  constexpr int NQ = 32 / RPR;    // ... read-backs per 32-row block
  constexpr int BM = 256, BN = 256;
  constexpr int STAGE = BM * kBK;   // 16 KiB of activations per K-step
  constexpr int DPW = STAGE / 1024 / 4;  // 1 KiB direct-to-LDS loads per wavefront per stage
  constexpr int BPW = 2 * WNB;           // weight fragment loads per wavefront per step
  constexpr int G = DPW + BPW;           // vector-memory ops per wavefront per step
  // EPI_PLAIN16 / EPI_BIAS16: 16-bit outputs without / with bias; EPI_GENERAL: fp32 outputs; EPI_ACC: any output
  // with the accumulator dump (the last two handle bias at run time)
  constexpr bool STAGED = ODT != H3K_F32;
  constexpr bool ACC = EPI == EPI_ACC;
  constexpr bool FAST = EPI == EPI_PLAIN16 || EPI == EPI_BIAS16;
  static_assert(!FAST || STAGED, "the 16-bit epilogue needs a 16-bit output");
  static_assert(LAY == 0 || FAST, "the fp32 and accumulator-dump epilogues assume 2 x 2 wavefronts");
  constexpr int NEPI = NQ * WMB;         // stores of one full-tile 16-bit epilogue per wavefront
  constexpr int GROW = WCOLS + 4;        // staging row pitch: a wavefront's columns + 4 32-bit values of padding
  constexpr int RS = 2;                  // scale slots (tile t uses slot t % 2)
  constexpr int SLOT = 768;              // floats per slot: 256 xs, 256 s_ch, then 1 KiB of bias
  constexpr int BES = ODT == H3K_F32 ? 4 : 2;  // bias element bytes (the output dtype)
  constexpr int STEADY = G * (S - 2);
  static_assert(STEADY + NEPI + 1 < 64, "vmcnt allowance out of range");
  // staging words per wavefront: two 32-row blocks on 1 x 4 wavefronts (double-buffered 16-bit epilogue), one on 2 x 2
  constexpr int STG_WORDS = (LAY ? 2 : 1) * 32 * GROW;
  __shared__ __attribute__((aligned(1024))) int8_t smem[S * STAGE + RS * SLOT * 4 + 4 * STG_WORDS * 4];
  float* const sscale = reinterpret_cast<float*>(smem + S * STAGE);

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int NG = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
  // Items of this workgroup: the whole tiles bid, bid + NG, ... below tiles_dp, then (split tail, 16-bit outputs
  // only) piece bid of the tiles from tiles_dp on: tail tile bid / P, K-steps [(bid % P) KP, (bid % P + 1) KP),
  // whose int32 partial sums go to part[bid] for w8p_fixup_kernel.
  const int T_dp = bid < tiles_dp ? (tiles_dp - bid + NG - 1) / NG : 0;
  const bool piece = FAST && P > 1 && bid < (tiles - tiles_dp) * P;
  const int T = T_dp + (piece ? 1 : 0);
  if (T == 0) return;  // the whole workgroup: nothing was issued yet
  const int KT = K / kBK;  // a multiple of S, >= 2 * S (host); KP likewise
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = LAY ? 0 : wave >> 1, wn = LAY ? wave : wave & 1;
  const int kh = lane >> 5;

  // item it -> tile origin, first K-step and K-step count
  auto coords = [&](int it, int& m0, int& n0, int& k0, int& kt) {
    int t = bid + it * NG;
    k0 = 0;
    kt = KT;
    if (FAST && it >= T_dp) {
      t = tiles_dp + bid / P;
      k0 = (bid % P) * KP;
      kt = KP;
    }
    int tm, tn;
    tile_coords<kTileGroupRows>(t, tiles_m, tiles_n, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
  };

  // ---------------------------------------------------------------- load streams
  // Activations: buffer loads straight to LDS (one 32-bit row offset per load, the K position in a scalar).
  // Weights: buffer loads into registers, issued as inline assembly -- see weight_load -- and covered by the
  // explicit waits before each barrier.  The K loop carries few scalars: the next tile's origin is computed at tile
  // start, not inside the loop.
  const rsrc_t ra = make_rsrc(A, static_cast<uint32_t>(static_cast<int64_t>(M - 1) * lda + K));
  const u32x4 rb = weight_rsrc(Bp, bp_bytes);
  const uint32_t bvoff = static_cast<uint32_t>(lane) * 16u;
  const uint32_t bstride = static_cast<uint32_t>(NBP) * kBlockBytes;  // one K-step of the packed grid
  uint32_t aoff[DPW];   // this lane's 16-byte chunk of each of its DPW activation rows (K position 0)
  uint32_t astep = 0;   // activations: K position of the next stage to load, in bytes
  uint32_t bnext = 0;   // weights: offset of this wavefront's 4 blocks at the next K-step to load
  uint32_t bfirst = 0;  // ... and at K-step 0 of the tile being loaded (a safe address for the tail loads)
  auto point_loads = [&](int m0, int n0, int k0) {
    // recomputed from an opaque lane index each time: kept from the prologue, these would be spilled
    int l = static_cast<int>(threadIdx.x & 63);
    __asm__ volatile("" : "+v"(l));
    static_for<DPW>([&](auto i) {
      const int r = (wave * DPW + i) * 16 + (l >> 2);  // (M - 1) * lda + K < 2^32 (host)
      aoff[i] = static_cast<uint32_t>(min(m0 + r, M - 1)) * static_cast<uint32_t>(lda) +
                static_cast<uint32_t>(swz_chunk(r, l & 3) * 16);
    });
    bfirst = static_cast<uint32_t>((n0 >> 5) + wn * WNB) * kBlockBytes;
    bnext = FAST ? bfirst + static_cast<uint32_t>(k0) * bstride : bfirst;
    astep = FAST ? static_cast<uint32_t>(k0) * kBK : 0u;
  };
  // Waves 0, 1 and 2 load the tile's 256 xs, 256 s_ch and 256 bias values, one 16-byte chunk per lane.  A chunk
  // past the end of its array is clamped to the 16-byte chunk that holds the last element (the arrays are 16-byte
  // aligned, so that chunk lies in the same page as the element): the values it brings are those of rows or
  // columns that are never stored.  Every stored row and column therefore reads its own value from the slot.
  auto load_scales = [&](int slot, int m0, int n0) {
    float* const dst = sscale + slot * SLOT + wave * 256;
    if (wave == 0) {
      const int r = min(m0 + 4 * lane, (M - 1) & ~3);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(xs + r), (lds_void*)dst, 16, 0, 0);
    } else if (wave == 1) {
      const int c = min(n0 + 4 * lane, (N - 1) & ~3);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(sch + c), (lds_void*)dst, 16, 0, 0);
    } else if (EPI == EPI_BIAS16 && wave == 2 && lane * (16 / BES) < BN) {
      constexpr int PER = 16 / BES;  // bias values per chunk
      const int c = min(n0 + PER * lane, (N - 1) / PER * PER);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(static_cast<const char*>(bias) + c * BES),
                                       (lds_void*)dst, 16, 0, 0);
    }
  };
  // Every step issues the same G vector-memory ops: after the last step of the last tile the loads re-read K
  // position 0 into a stage and registers nobody reads again, so the wait counts never depend on the path.
  auto issue_a = [&](int stage, bool real) {
    int8_t* dst = smem + stage * STAGE + wave * DPW * 1024;
    const uint32_t k = real ? astep : 0u;
    static_for<DPW>([&](auto i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(dst + i * 1024), 16, static_cast<int>(aoff[i]),
                                                static_cast<int>(k), 0, 0);
    });
    astep += kBK;
  };
  v4i bq[S][WNB][2];  // weight fragments of S steps
  auto issue_b = [&](auto u, bool real) {
    // values, not a conditional lvalue: a select between the two variables' addresses would keep both in memory
    const uint32_t bn = bnext, bf = bfirst;
    const uint32_t b0 = real ? bn : bf, b1 = b0 + 4096u;  // blocks 0-1 and 2-3: 12-bit immediate offsets
    static_for<WNB>([&](auto j) {
      constexpr int J = decltype(j)::value;
      weight_load<(J % 2) * 2048>(bq[u][J][0], rb, bvoff, J < 2 ? b0 : b1);
      weight_load<(J % 2) * 2048 + 1024>(bq[u][J][1], rb, bvoff, J < 2 ? b0 : b1);
    });
    bnext += bstride;
  };

  // ---------------------------------------------------------------- fragments and MFMA
  const int arow = wm * WROWS + (lane & 31);
  auto read_frags = [&](int stage, int half, v4i (&af)[WMB]) {
    const int8_t* base = smem + stage * STAGE;
    const int c = kh * 2 + half;  // the packed weight's k order: lanes 32-63 own the step's last 32 bytes
    static_for<WMB>([&](auto i) { af[i] = *reinterpret_cast<const v4i*>(base + swz(arow + i * 32, c)); });
  };
  v16i acc[WMB][WNB];
  auto mfma = [&](const v4i (&af)[WMB], auto u, auto h) {
    static_for<WMB>([&](auto i) {
      static_for<WNB>([&](auto j) {
        // weights as the first operand: each lane's accumulators hold one output row (see the epilogue)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bq[u][j][h], af[i], acc[i][j], 0, 0, 0);
      });
    });
  };

  // ---------------------------------------------------------------- epilogue
  // Lane l owns output row m = cm0 + wm * WROWS + i * 32 + (l & 31) (i < WMB) and, per j < WNB, the columns
  // cn0 + wn * WCOLS + j * 32 + g * 8 + (l >> 5) * 4 + e (g, e < 4).
  int cm0 = 0, cn0 = 0;
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  auto scaled = [&](int a, float x, float s) -> float {
    return value_point(EAGER ? static_cast<float>(a) * value_point(x * s) : value_point(static_cast<float>(a) * x) * s);
  };
  auto bits16 = [&](float f) -> uint32_t { return ODT == H3K_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); };
  auto round16 = [&](float f) -> float { return ODT == H3K_F16 ? round_f16(f) : round_bf16(f); };
  auto pack4 = [&](const float (&f)[4]) -> uint2 {
    if (ODT == H3K_BF16) {
      const bf16x2 lo = __builtin_convertvector((f32x2){f[0], f[1]}, bf16x2);
      const bf16x2 hi = __builtin_convertvector((f32x2){f[2], f[3]}, bf16x2);
      return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    }
    return make_uint2(bits16(f[0]) | (bits16(f[1]) << 16), bits16(f[2]) | (bits16(f[3]) << 16));
  };

  // Stores the finished tile; true when exactly NEPI vector-memory ops were issued (a whole 16-bit tile).
  // Per 32-row block, the wavefront writes its accumulators into its staging area and reads them back
  // row-contiguous, 8 columns per lane.
  //   16-bit outputs: the raw int32 accumulators go through the staging area; the scale (and bias) of a lane's 8
  //   columns are the same for every row, so they are read from the tile's slot once, and each row's xs is one
  //   LDS read.  Rows inside M store 8 outputs as one 16-byte non-temporal store when the output rows are 16-byte
  //   aligned and the 8 columns lie inside N, else element by element.  Nothing here waits for vector memory: the
  //   next tile's loads stay in flight.
  //   fp32 outputs or the accumulator dump: fp32 results (and the raw accumulators) are staged and stored 4 per
  //   lane after waiting for every load in flight -- the next tile's weight fragments included, so nothing in
  //   flight can be spilled there.
  // One path per instantiation keeps the accumulator reads to one block at a time.
  auto epilogue = [&](int slot) -> bool {
    // lane- and tile-derived values recomputed from opaque copies: shared with the K loop's address arithmetic
    // they would stay live across it
    int lane = static_cast<int>(threadIdx.x & 63);
    __asm__ volatile("" : "+v"(lane));
    const int kh = lane >> 5;
    const float* const sx = sscale + slot * SLOT;
    float* const stg = reinterpret_cast<float*>(smem + S * STAGE + RS * SLOT * 4) + wave * STG_WORDS;
    if constexpr (FAST) {
      const int c8 = wn * WCOLS + (lane % LPR) * 8;  // the lane's 8 columns, relative to the tile
      const int gcol = cn0 + c8;
      const bool lines = (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (ldo & 7) == 0;
      const bool cols_in = gcol + 8 <= N;
      const bool whole = lines && cm0 + BM <= M && cn0 + BN <= N;  // every store a whole 16-byte vector
      float sc[8], bv[8];
      {
        // element reads of the slot: a 16-byte LDS read of memory a direct-to-LDS load wrote makes the compiler
        // wait for vmcnt(0), i.e. for the next tile's loads in flight
        static_for<8>([&](auto e) { sc[e] = sx[256 + c8 + e]; });
        if constexpr (EPI == EPI_BIAS16) {
          const uint32_t* const b = reinterpret_cast<const uint32_t*>(sx + 512) + c8 / 2;  // 8 16-bit values
          static_for<4>([&](auto e) {
            const uint32_t two = b[e];
            bv[2 * e] = ODT == H3K_F16 ? f16_to_f32(two & 0xFFFFu) : bf16_to_f32(two & 0xFFFFu);
            bv[2 * e + 1] = ODT == H3K_F16 ? f16_to_f32(two >> 16) : bf16_to_f32(two >> 16);
          });
        }
      }
      if (LAY && whole) {
        // The 32-row blocks through two staging buffers: block i + 1's accumulators go to LDS right after block i's
        // read-back is issued, so those writes (the slower LDS direction) overlap block i's arithmetic.
        int32_t* const sb0 = reinterpret_cast<int32_t*>(stg);
        int32_t* const sb1 = sb0 + 32 * GROW;
        auto stage_blk = [&](auto i, int32_t* buf) {
          int32_t* const w = buf + (lane & 31) * GROW + kh * 4;
          static_for<WNB>([&](auto j) {
            static_for<4>([&](auto g) {
              *reinterpret_cast<v4i*>(w + j * 32 + g * 8) =
                  v4i{acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
            });
          });
        };
        stage_blk(std::integral_constant<int, 0>{}, sb0);
        static_for<WMB>([&](auto i) {
          constexpr int I = decltype(i)::value;
          __builtin_amdgcn_sched_barrier(0);
          wave_lds_sync();
          const int32_t* const rp = (I % 2 ? sb1 : sb0) + (lane / LPR) * GROW + (lane % LPR) * 8;
          const float* const xr = sx + wm * WROWS + I * 32 + lane / LPR;
          v4i lo[NQ], hi[NQ];
          float x[NQ];
          static_for<NQ>([&](auto q) {
            lo[q] = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW);
            hi[q] = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW + 4);
            x[q] = xr[q * RPR];
          });
          if constexpr (I + 1 < WMB) stage_blk(std::integral_constant<int, I + 1>{}, (I + 1) % 2 ? sb1 : sb0);
          uint16_t* const obase = static_cast<uint16_t*>(out) +
                                  static_cast<int64_t>(cm0 + wm * WROWS + I * 32 + lane / LPR) * ldo + gcol;
          static_for<NQ>([&](auto q) {
            const int a[8] = {lo[q][0], lo[q][1], lo[q][2], lo[q][3], hi[q][0], hi[q][1], hi[q][2], hi[q][3]};
            float f[8];
            static_for<8>([&](auto e) {
              float y = scaled(a[e], x[q], sc[e]);
              if constexpr (EPI == EPI_BIAS16)  // added after the output rounding (qlinear.py:404-405)
                y = value_point(round16(y) + bv[e]);
              f[e] = y;
            });
            const uint2 p0 = pack4({f[0], f[1], f[2], f[3]}), p1 = pack4({f[4], f[5], f[6], f[7]});
            __builtin_nontemporal_store(u32x4{p0.x, p0.y, p1.x, p1.y},
                                        reinterpret_cast<u32x4*>(obase + static_cast<int64_t>(q * RPR) * ldo));
          });
        });
        wave_lds_sync();  // the staging area is free before the next epilogue
        return true;
      }
      static_for<WMB>([&](auto i) {
        __builtin_amdgcn_sched_barrier(0);
        int32_t* const w = reinterpret_cast<int32_t*>(stg) + (lane & 31) * GROW + kh * 4;
        static_for<WNB>([&](auto j) {
          static_for<4>([&](auto g) {
            *reinterpret_cast<v4i*>(w + j * 32 + g * 8) =
                v4i{acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
          });
        });
        wave_lds_sync();
        const float* const xr = sx + wm * WROWS + i * 32 + lane / LPR;
        // the 8 outputs of row q * RPR + lane / LPR of the block at the lane's 8 columns, from its raw accumulators
        auto row_out = [&](const v4i& lo, const v4i& hi, float x, float (&f)[8]) {
          const int a[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          static_for<8>([&](auto e) {
            float y = scaled(a[e], x, sc[e]);
            if constexpr (EPI == EPI_BIAS16)  // added after the output rounding (qlinear.py:404-405)
              y = value_point(round16(y) + bv[e]);
            f[e] = y;
          });
        };
        const int32_t* const rp = reinterpret_cast<const int32_t*>(stg) + (lane / LPR) * GROW + (lane % LPR) * 8;
        const int row_b = cm0 + wm * WROWS + i * 32 + lane / LPR;  // the lane's row for q = 0
        uint16_t* const obase = static_cast<uint16_t*>(out) + static_cast<int64_t>(row_b) * ldo + gcol;
        if (whole) {
          // the accumulators of RB rows read first (8 RB registers): the LDS latency is paid once per batch, and
          // no branch splits the arithmetic and the stores.  With bias, whose 8 values take registers too, batches
          // of 4 rows keep the epilogue from spilling the next tile's weight registers.
          constexpr int RB = EPI == EPI_BIAS16 ? 4 : (NQ < 8 ? NQ : 8);
          static_for<NQ / RB>([&](auto bt) {
            v4i lo[RB], hi[RB];
            float x[RB];
            static_for<RB>([&](auto r) {
              constexpr int q = decltype(bt)::value * RB + decltype(r)::value;
              lo[r] = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW);
              hi[r] = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW + 4);
              x[r] = xr[q * RPR];
            });
            static_for<RB>([&](auto r) {
              constexpr int q = decltype(bt)::value * RB + decltype(r)::value;
              float f[8];
              row_out(lo[r], hi[r], x[r], f);
              const uint2 p0 = pack4({f[0], f[1], f[2], f[3]}), p1 = pack4({f[4], f[5], f[6], f[7]});
              __builtin_nontemporal_store(u32x4{p0.x, p0.y, p1.x, p1.y},
                                          reinterpret_cast<u32x4*>(obase + static_cast<int64_t>(q * RPR) * ldo));
            });
          });
        } else {
          static_for<NQ>([&](auto q) {
            const v4i lo = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW);
            const v4i hi = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW + 4);
            float f[8];
            row_out(lo, hi, xr[q * RPR], f);
            if (row_b + q * RPR < M) {
              uint16_t* const orow = obase + static_cast<int64_t>(q * RPR) * ldo;
              if (lines && cols_in) {
                const uint2 p0 = pack4({f[0], f[1], f[2], f[3]}), p1 = pack4({f[4], f[5], f[6], f[7]});
                *reinterpret_cast<u32x4*>(orow) = u32x4{p0.x, p0.y, p1.x, p1.y};
              } else {
                static_for<8>([&](auto e) {
                  if (gcol + e < N) orow[e] = static_cast<uint16_t>(bits16(f[e]));
                });
              }
            }
          });
        }
        wave_lds_sync();  // the next block overwrites the staging area
      });
      return whole;
    } else {
      const int row0 = cm0 + wm * 128 + (lane & 31);
      const int col0 = cn0 + wn * 128 + kh * 4;
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<0>();
      __builtin_amdgcn_sched_barrier(0);
      static_for<WMB>([&](auto i) {
        static_for<2>([&](auto pass) {  // 0: outputs, 1: accumulators (acc_out)
          if (pass == 1 && !ACC) return;
          __builtin_amdgcn_sched_barrier(0);
          const float x = sx[row0 - cm0 + i * 32];
          float* const w = stg + (lane & 31) * GROW + kh * 4;
          static_for<WNB>([&](auto j) {
            static_for<4>([&](auto g) {
              // element reads of the scale slot: a 16-byte LDS read here makes the compiler drain vmcnt
              const float* p = sx + 256 + col0 - cn0 + j * 32 + g * 8;
              float4 v;
              if (pass == 0) {
                v = make_float4(scaled(acc[i][j][g * 4 + 0], x, p[0]), scaled(acc[i][j][g * 4 + 1], x, p[1]),
                                scaled(acc[i][j][g * 4 + 2], x, p[2]), scaled(acc[i][j][g * 4 + 3], x, p[3]));
              } else {
                v = make_float4(__int_as_float(acc[i][j][g * 4 + 0]), __int_as_float(acc[i][j][g * 4 + 1]),
                                __int_as_float(acc[i][j][g * 4 + 2]), __int_as_float(acc[i][j][g * 4 + 3]));
              }
              *reinterpret_cast<float4*>(w + j * 32 + g * 8) = v;
            });
          });
          wave_lds_sync();
          const int r2 = lane >> 5, c4 = (lane & 31) * 4;  // rows r2 + 2q, columns c4 .. c4 + 3 of the block
          const int n = cn0 + wn * 128 + c4;
          static_for<16>([&](auto q) {
            const int m = cm0 + wm * 128 + i * 32 + r2 + 2 * q;
            const float4 v = *reinterpret_cast<const float4*>(stg + (r2 + 2 * q) * GROW + c4);
            if (m < M) {
              const float f[4] = {v.x, v.y, v.z, v.w};
              if (pass == 1) {
                int32_t* dst = acc_out + static_cast<int64_t>(m) * N + n;
                static_for<4>([&](auto e) {
                  if (n + e < N) dst[e] = __float_as_int(f[e]);
                });
              } else {
                float o[4];
                static_for<4>([&](auto e) {
                  float y = f[e];
                  if (ODT != H3K_F32) y = round16(y);
                  if (bias && n + e < N) {  // added after the output rounding (qlinear.py:404-405)
                    float b;
                    if (ODT == H3K_F32) b = static_cast<const float*>(bias)[n + e];
                    else if (ODT == H3K_F16) b = f16_to_f32(static_cast<const uint16_t*>(bias)[n + e]);
                    else b = bf16_to_f32(static_cast<const uint16_t*>(bias)[n + e]);
                    y = ODT == H3K_F32 ? y + b : fp32_round_point(y + b);
                  }
                  o[e] = y;
                });
                const int64_t off = static_cast<int64_t>(m) * ldo + n;
                if (n + 3 < N && vec_out) {
                  if (ODT == H3K_F32)
                    *reinterpret_cast<float4*>(static_cast<float*>(out) + off) = make_float4(o[0], o[1], o[2], o[3]);
                  else
                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + off) =
                        make_uint2(bits16(o[0]) | (bits16(o[1]) << 16), bits16(o[2]) | (bits16(o[3]) << 16));
                } else {
                  static_for<4>([&](auto e) {
                    if (n + e < N) {
                      if (ODT == H3K_F32) static_cast<float*>(out)[off + e] = o[e];
                      else static_cast<uint16_t*>(out)[off + e] = static_cast<uint16_t>(bits16(o[e]));
                    }
                  });
                }
              }
            }
          });
          wave_lds_sync();  // the next block overwrites the staging area
        });
      });
      wait_vmcnt<0>();  // nothing of unknown count stays pending into the next tile's first steps
      return false;
    }
  };

  // A piece's int32 partial sums, row-major [256][256] at part[bid], through the staging area: each lane reads 8
  // consecutive columns of a row back, so the 16 lanes of a row store its 128 columns of this wavefront as 512
  // contiguous bytes.
  auto dump_partial = [&]() {
    if constexpr (FAST) {
      int lane = static_cast<int>(threadIdx.x & 63);
      __asm__ volatile("" : "+v"(lane));
      const int kh = lane >> 5;
      int32_t* const stg = reinterpret_cast<int32_t*>(smem + S * STAGE + RS * SLOT * 4) + wave * STG_WORDS;
      int32_t* const dst = part + static_cast<int64_t>(bid) * (BM * BN);
      static_for<WMB>([&](auto i) {
        __builtin_amdgcn_sched_barrier(0);
        int32_t* const w = stg + (lane & 31) * GROW + kh * 4;
        static_for<WNB>([&](auto j) {
          static_for<4>([&](auto g) {
            *reinterpret_cast<v4i*>(w + j * 32 + g * 8) =
                v4i{acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
          });
        });
        wave_lds_sync();
        const int32_t* const rp = stg + (lane / LPR) * GROW + (lane % LPR) * 8;
        static_for<NQ>([&](auto q) {
          const v4i lo = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW);
          const v4i hi = *reinterpret_cast<const v4i*>(rp + q * RPR * GROW + 4);
          int32_t* const o = dst + (wm * WROWS + i * 32 + q * RPR + lane / LPR) * BN + wn * WCOLS + (lane % LPR) * 8;
          *reinterpret_cast<v4i*>(o) = lo;
          *reinterpret_cast<v4i*>(o + 4) = hi;
        });
        wave_lds_sync();  // the next block overwrites the staging area
      });
    }
  };

  // ---------------------------------------------------------------- prologue
  int ck0 = 0, ckt = KT;  // the current item's first K-step and K-step count
  coords(0, cm0, cn0, ck0, ckt);
  point_loads(cm0, cn0, ck0);
  load_scales(0, cm0, cn0);
  static_for<S>([&](auto s) {
    issue_a(s, true);
    issue_b(s, true);
  });
  wait_vmcnt<G * (S - 1)>();
  lds_barrier();

  v4i a0[WMB], a1[WMB];
  read_frags(0, 0, a0);
  bool exact = false;  // the last epilogue issued exactly NEPI vector-memory ops
  bool has_next = false;
  int it = 0;

  // One K-step in stage u.  FIRST: the tile's first step, whose first MFMAs start from zero (no accumulator
  // clearing between tiles).  WAIT: which allowance the wait before the barrier uses -- step kt + 1 must have
  // landed; normally the S - 2 newer steps may still be in flight (W_STEADY); in the S - 1 steps after an epilogue
  // its stores (and the scale loads) sit in between (W_AFTER_EPI); in the last tile's last steps wait for everything
  // (W_TAIL), or for everything without issuing loads (W_DRAIN: the last steps of a tile whose epilogue does not
  // run across the next tile's loads).  more: step kt + S exists (this tile's or the next one's); frags: step
  // kt + 1 is this tile's.  The steady steps have every choice fixed at compile time: no branch interrupts their
  // MFMA stream.
  enum { W_STEADY = 0, W_AFTER_EPI = 1, W_TAIL = 2, W_DRAIN = 3 };
  auto step = [&](auto u, auto first, auto wait, bool more, bool frags) {
    read_frags(u, 1, a1);
    if constexpr (first.value) {
      static_for<WMB>([&](auto i) {
        static_for<WNB>([&](auto j) { acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bq[u][j][0], a0[i], v16i{}, 0, 0, 0); });
      });
    } else {
      mfma(a0, u, std::integral_constant<int, 0>{});
    }
    // The scheduling region runs from the last barrier to here: the previous step's second half (its MFMAs, the
    // first DPW of them each behind one activation DMA issue, then this step's first-half fragment reads one per
    // MFMA) and this step's first half (its MFMAs, kEarlyMfma of them ahead of the second-half reads, then one read
    // per MFMA).  Pinning the whole region keeps the second-half reads from sinking to the wait before the barrier,
    // where the compiler's own order had put them, and the DMA issues (each behind an M0 write) from holding back
    // the first MFMAs after the barrier.
    static_for<DPW>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read: one activation DMA issue per MFMA
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    });
    static_for<WMB>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    });
    __builtin_amdgcn_sched_group_barrier(0x008, WMB * WNB - DPW - WMB, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, kEarlyMfma, 0);
    static_for<WMB>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    });
    __builtin_amdgcn_sched_group_barrier(0x008, WMB * WNB - kEarlyMfma - WMB, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
    if constexpr (wait.value == W_STEADY) {
      wait_vmcnt<STEADY>();
    } else if constexpr (wait.value == W_AFTER_EPI) {
      if (it == 0) wait_vmcnt<STEADY>();
      else if (exact) wait_vmcnt<STEADY + NEPI>();
      else wait_vmcnt<0>();
    } else if constexpr (wait.value == W_TAIL) {
      if (has_next) wait_vmcnt<STEADY>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if constexpr (wait.value != W_DRAIN) issue_a(u, more);  // stage kt + S into the stage just read
    if (frags) read_frags((u + 1) % S, 0, a0);
    mfma(a1, u, std::integral_constant<int, 1>{});
    if constexpr (wait.value != W_DRAIN) issue_b(u, more);  // weight fragments of step kt + S into the registers just consumed
  };
  // The 16-bit epilogue runs with the next tile's first S steps of loads in flight.  The fp32 and accumulator-dump
  // epilogues need more registers than that leaves: their tiles end with the load streams drained and start the
  // next tile's streams afresh, as the prologue does.
  constexpr bool CROSS = FAST;
  using std::integral_constant;
  for (; it < T; ++it) {
    has_next = it + 1 < T;
    int nm0 = 0, nn0 = 0, nk0 = 0, nkt = KT;  // the next item
    if (has_next) coords(it + 1, nm0, nn0, nk0, nkt);
    if (it > 0) {
      if constexpr (CROSS) {
        load_scales(it % RS, cm0, cn0);
      } else {
        point_loads(cm0, cn0, ck0);
        load_scales(it % RS, cm0, cn0);
        static_for<S>([&](auto s) {
          issue_a(s, true);
          issue_b(s, true);
        });
        wait_vmcnt<G * (S - 1)>();
        lds_barrier();
        read_frags(0, 0, a0);
      }
    }
    static_for<S>([&](auto u) {  // steps 0 .. S - 1 (K has at least 2 S steps)
      constexpr int U = decltype(u)::value;
      step(u, integral_constant<bool, U == 0>{}, integral_constant<int, U < S - 1 ? W_AFTER_EPI : W_STEADY>{}, true, true);
    });
    for (int kt0 = S; kt0 < (FAST ? ckt : KT) - S; kt0 += S) {
      static_for<S>([&](auto u) {
        step(u, integral_constant<bool, false>{}, integral_constant<int, W_STEADY>{}, true, true);
      });
    }
    if (CROSS && has_next) point_loads(nm0, nn0, nk0);  // the load streams move on to the next item
    static_for<S>([&](auto u) {  // steps KT - S .. KT - 1
      step(u, integral_constant<bool, false>{}, integral_constant<int, CROSS ? W_TAIL : W_DRAIN>{}, has_next,
           decltype(u)::value < S - 1);
    });
    if (piece && it == T - 1) {
      dump_partial();  // the last item: nothing is in flight behind it
    } else {
      exact = epilogue(it % RS);
    }
    if (has_next) {
      if constexpr (CROSS) read_frags(0, 0, a0);
      cm0 = nm0;
      cn0 = nn0;
      ck0 = nk0;
      ckt = nkt;
    }
  }
  wait_vmcnt<0>();  // no direct-to-LDS write may land after the workgroup has ended
}

constexpr int kW8pS = 4;  // steps of the weight register ring and the activation LDS ring

// Split tail: the int32 partial sums of the P pieces of each tail tile added in a fixed order (exact), then the
// kernel's 16-bit epilogue.  One workgroup per 16 rows of a tail tile; a thread owns 16 consecutive columns of a row,
// so a row's 256 partial sums are 1 KiB contiguous per piece.
template <int ODT, bool EAGER>
__global__ __launch_bounds__(256) void w8p_fixup_kernel(const int32_t* __restrict__ part, int P, int tiles_dp, int M,
                                                        int N, const float* __restrict__ xs,
                                                        const float* __restrict__ sch, const void* __restrict__ bias,
                                                        uint16_t* __restrict__ out, int64_t ldo, bool vec_out) {
  constexpr int BM = 256, BN = 256;
  const int tt = static_cast<int>(blockIdx.x) >> 4, rg = static_cast<int>(blockIdx.x) & 15;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords<kTileGroupRows>(tiles_dp + tt, tiles_m, tiles_n, tm, tn);
  const int r = rg * 16 + static_cast<int>(threadIdx.x >> 4), c = static_cast<int>(threadIdx.x & 15) * 16;
  const int m = tm * BM + r, n0 = tn * BN + c;
  if (m >= M || n0 >= N) return;
  int a[16];
  for (int e = 0; e < 16; ++e) a[e] = 0;
  for (int p = 0; p < P; ++p) {
    const v4i* src = reinterpret_cast<const v4i*>(part + (static_cast<int64_t>(tt) * P + p) * (BM * BN) + r * BN + c);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const v4i x = __builtin_nontemporal_load(src + v);
      a[4 * v] += x[0];
      a[4 * v + 1] += x[1];
      a[4 * v + 2] += x[2];
      a[4 * v + 3] += x[3];
    }
  }
  const float x = xs[m];
  uint32_t bits[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int n = min(n0 + e, N - 1);  // columns past N are computed on the last one and never stored
    const float sc = sch[n];
    float y = EAGER ? value_point(static_cast<float>(a[e]) * value_point(x * sc))
                    : value_point(value_point(static_cast<float>(a[e]) * x) * sc);
    if (bias) {  // added after the output rounding (qlinear.py:404-405)
      const uint32_t b = static_cast<const uint16_t*>(bias)[n];
      const float rb = ODT == H3K_F16 ? round_f16(y) : round_bf16(y);
      y = value_point(rb + (ODT == H3K_F16 ? f16_to_f32(b) : bf16_to_f32(b)));
    }
    bits[e] = ODT == H3K_F16 ? f32_to_f16_bits(y) : f32_to_bf16_bits(y);
  }
  uint16_t* const o = out + static_cast<int64_t>(m) * ldo + n0;
  if (vec_out && n0 + 16 <= N) {
    u32x4 w0, w1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w0[e] = bits[2 * e] | (bits[2 * e + 1] << 16);
      w1[e] = bits[8 + 2 * e] | (bits[8 + 2 * e + 1] << 16);
    }
    reinterpret_cast<u32x4*>(o)[0] = w0;
    reinterpret_cast<u32x4*>(o)[1] = w1;
  } else {
    for (int e = 0; e < 16 && n0 + e < N; ++e) o[e] = static_cast<uint16_t>(bits[e]);
  }
}

template <int ODT, bool EAGER, int EPI>
static void launch(const int8_t* a, int64_t lda, const int8_t* bp, uint32_t bp_bytes, int nbp, int m, int n, int k,
                   const float* xs, const float* sch, const void* bias, void* out, int64_t ldo, int32_t* acc, int grid,
                   int tiles_dp, int P, int KP, int32_t* part, hipStream_t st) {
  const size_t es = ODT == H3K_F32 ? 4 : 2;
  const bool vec_out = aligned(out, 4 * es) && ldo % 4 == 0;
  // 16-bit epilogues: 1 x 4 wavefronts (no weight fragment loaded twice: 0.9 % faster at the headline shape)
  constexpr int LAY = (EPI == EPI_PLAIN16 || EPI == EPI_BIAS16) ? 1 : 0;
  hipLaunchKernelGGL((gemm_w8p_kernel<kW8pS, ODT, EAGER, EPI, LAY>), dim3(grid), dim3(256), 0, st, a, lda, bp, bp_bytes,
                     nbp, m, n, k, xs, sch, bias, out, ldo, acc, vec_out, tiles_dp, P, KP, part);
  if constexpr (ODT != H3K_F32 && (EPI == EPI_PLAIN16 || EPI == EPI_BIAS16)) {
    const int tiles = ((m + 255) / 256) * ((n + 255) / 256);
    if (P > 1)
      hipLaunchKernelGGL((w8p_fixup_kernel<ODT, EAGER>), dim3((tiles - tiles_dp) * 16), dim3(256), 0, st, part, P,
                         tiles_dp, m, n, xs, sch, bias, static_cast<uint16_t*>(out), ldo,
                         aligned(out, 16) && ldo % 8 == 0);
  }
}

// ------------------------------------------------------------------------------------------ packing
// Row-major int8 grid [n, k] -> packed layout.  One thread per 16-byte fragment chunk, in packed order: a
// wavefront's stores are 1 KiB contiguous.  Rows past n are written as zeros.
__global__ __launch_bounds__(256) void pack_w8_kernel(const int8_t* __restrict__ w8, int64_t ldw, int n, int nbp,
                                                      int8_t* __restrict__ wp, int64_t chunks) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= chunks) return;
  const int l = static_cast<int>(u & 63);
  const int64_t frag = u >> 6;  // (t * NBP + b) * 2 + h
  const int h = static_cast<int>(frag & 1);
  const int64_t tb = frag >> 1;
  const int b = static_cast<int>(tb % nbp);
  const int t = static_cast<int>(tb / nbp);
  const int row = b * 32 + (l & 31);
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (row < n) v = *reinterpret_cast<const u32x4*>(w8 + static_cast<int64_t>(row) * ldw + t * 64 + (l >> 5) * 32 + h * 16);
  *reinterpret_cast<u32x4*>(wp + u * 16) = v;
}

}  // namespace w8p

int cu_count();

// Bytes of the packed grid of an [n, k] weight (n padded to a multiple of 256: a whole output tile).
int64_t w8p_bytes(int64_t n, int64_t k) { return (n + 255) / 256 * 256 * k; }

// Work split of the persistent launch, and its cost in K-steps of a 256 x 256 tile (the model below, fitted to
// the config-3 shapes on MI355X: a K-step ~0.8 us of one round, the split tail's partial sums ~1.1 steps per MiB
// written and read back, ~6 steps for the fix-up launch).  Whole rounds of tiles run data-parallel (one workgroup
// per CU).  When the last round would leave CUs idle, its `rem` tiles may be cut into P pieces of KT / P K-steps
// each (P the largest that fits rem * P <= CUs, with pieces of whole S-step groups and at least 2 S steps), and a
// fix-up kernel adds each tile's P partial sums: taken where the model says it is faster.  P = 1: no split.
struct W8pPlan {
  int grid, tiles_dp, P, KP;
  int64_t part_bytes;
  double steps;  // modelled time in tile K-steps
};
static W8pPlan w8p_plan(int64_t m, int64_t n, int64_t k) {
  constexpr int S = w8p::kW8pS;
  const int cus = cu_count();
  const int tiles = static_cast<int>(((m + 255) / 256) * ((n + 255) / 256));
  const int kt = static_cast<int>(k / 64);
  const int rounds = tiles / cus, rem = tiles - rounds * cus;
  W8pPlan pl{tiles < cus ? tiles : cus, tiles, 1, kt, 0, static_cast<double>((rounds + (rem > 0)) * kt)};
  if (rem == 0) return pl;
  for (int p = cus / rem; p >= 2; --p) {
    if (kt % p == 0 && (kt / p) % S == 0 && kt / p >= 2 * S) {
      const int64_t part = static_cast<int64_t>(rem) * p * 256 * 256 * 4;
      const double steps = static_cast<double>(rounds) * kt + kt / p + 1.1 * static_cast<double>(part) / (1 << 20) + 6.0;
      if (steps < pl.steps) pl = W8pPlan{rounds > 0 ? cus : rem * p, rounds * cus, p, kt / p, part, steps};
      break;
    }
  }
  return pl;
}

// The shapes the kernel can run at all: K a multiple of 64 * S with at least 2 * S steps (the per-tile step phases
// must not overlap), M >= 4, N a multiple of 4, the packed grid addressable by one buffer descriptor.
static bool w8p_runs(int64_t m, int64_t n, int64_t k) {
  constexpr int S = w8p::kW8pS;
  if (k % (64 * S) || k < 2 * S * 64 || m < 4 || n < 4 || n % 4 || m > (1 << 30) || n > (1 << 30) || k > (1 << 17)) return false;
  return w8p_bytes(n, k) < (int64_t(1) << 32);
}

// Whether the W4A8 linear takes this kernel for the shape: one it runs, more than 512 rows, at least 5/8 of the CUs
// get a 256 x 256 tile, and its modelled time (with the split tail where that pays) is no worse than the row-major
// pipeline's on 128 x 256 tiles.
bool w8p_serves(int64_t m, int64_t n, int64_t k) {
  if (!w8p_runs(m, n, k)) return false;
  const int cus = cu_count();
  const int64_t tiles256 = ((m + 255) / 256) * ((n + 255) / 256), tiles128x256 = ((m + 127) / 128) * ((n + 255) / 256);
  if (m <= 512 || tiles256 < cus * 5 / 8) return false;
  // against the row-major pipeline on 128 x 256 tiles: half a tile's work per tile, at ~0.72 of this kernel's rate
  const double pipe = static_cast<double>((tiles128x256 + cus - 1) / cus) * static_cast<double>(k / 64) * 0.5 / 0.72;
  return w8p_plan(m, n, k).steps <= pipe;
}

// Preconditions (checked by the caller): w8p_serves(m, n, k); a and w8p 16-byte aligned, lda a multiple of 16;
// xs, s_ch and bias 16-byte aligned.
int64_t w8p_split_bytes(int64_t m, int64_t n, int64_t k) { return w8p_plan(m, n, k).part_bytes; }

// part: the split tail's partial sums (w8p_split_bytes), or nullptr for whole tiles only.  The split serves 16-bit
// outputs without the accumulator dump.
void gemm_w8p_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p, const float* s_ch,
                     const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo, int32_t* acc_out,
                     int32_t* part, hipStream_t st) {
  W8pPlan pl = w8p_plan(m, n, k);
  if (pl.P > 1 && (!part || acc_out || odt == H3K_F32)) {
    const int tiles = ((m + 255) / 256) * ((n + 255) / 256);
    pl = W8pPlan{tiles < cu_count() ? tiles : cu_count(), tiles, 1, k / 64, 0, 0.0};
  }
  const int grid = pl.grid;
  const uint32_t bytes = static_cast<uint32_t>(w8p_bytes(n, k));
  const int nbp = static_cast<int>((n + 255) / 256 * 8);
  const bool e = mode == H3K_MODE_EAGER;
#define H3K_L(D, E)                                                                                              \
  (e ? w8p::launch<D, true, E>(a, lda, w8p, bytes, nbp, m, n, k, xs, s_ch, bias, out, ldo, acc_out, grid,         \
                               pl.tiles_dp, pl.P, pl.KP, part, st)                                                \
     : w8p::launch<D, false, E>(a, lda, w8p, bytes, nbp, m, n, k, xs, s_ch, bias, out, ldo, acc_out, grid,        \
                                pl.tiles_dp, pl.P, pl.KP, part, st))
  // the accumulator dump has its own instantiations (a second read of every accumulator costs registers)
  if (odt == H3K_F32) {
    if (acc_out) H3K_L(H3K_F32, w8p::EPI_ACC); else H3K_L(H3K_F32, w8p::EPI_GENERAL);
  } else if (odt == H3K_F16) {
    if (acc_out) H3K_L(H3K_F16, w8p::EPI_ACC); else if (bias) H3K_L(H3K_F16, w8p::EPI_BIAS16); else H3K_L(H3K_F16, w8p::EPI_PLAIN16);
  } else {
    if (acc_out) H3K_L(H3K_BF16, w8p::EPI_ACC); else if (bias) H3K_L(H3K_BF16, w8p::EPI_BIAS16); else H3K_L(H3K_BF16, w8p::EPI_PLAIN16);
  }
#undef H3K_L
}

}  // namespace h3k

using namespace h3k;

extern "C" int64_t h3k_w8_packed_bytes(int64_t n, int64_t k) {
  if (n < 0 || k < 0 || k % 64) return -1;
  return w8p_bytes(n, k);
}

extern "C" int h3k_gemm_packed_serves(int64_t m, int64_t n, int64_t k) { return w8p_serves(m, n, k) ? 1 : 0; }

extern "C" int h3k_pack_w8(const int8_t* w8, int64_t ldw, int64_t n, int64_t k, int8_t* w8p, void* stream) {
  if (n < 0 || k <= 0 || k % 64 || k > (1 << 30) || n > (1 << 30)) return fail(H3K_EINVAL, "pack: bad n=%lld k=%lld (k a multiple of 64)", (long long)n, (long long)k);
  if (ldw < k) return fail(H3K_EINVAL, "row stride smaller than the rows");
  if (n == 0) return H3K_OK;
  if (!w8 || !w8p) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(w8, 16) || ldw % 16 || !aligned(w8p, 16)) return fail(H3K_EINVAL, "pack: 16-byte alignment needed");
  const int64_t chunks = w8p_bytes(n, k) / 16;
  hipLaunchKernelGGL(w8p::pack_w8_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w8, ldw, static_cast<int>(n),
                     static_cast<int>((n + 255) / 256 * 8), w8p, chunks);
  return check_launch("pack_w8");
}

extern "C" int h3k_gemm_a8w8_packed(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p, const float* s_ch,
                                    const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out,
                                    int out_dtype, int64_t ldo, int32_t* acc_out, void* stream) {
  if (m < 0 || n < 0 || k < 0) return fail(H3K_EINVAL, "bad GEMM shape");
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (out_dtype != H3K_BF16 && out_dtype != H3K_F16 && out_dtype != H3K_F32)
    return fail(H3K_EINVAL, "out dtype code %d unsupported", out_dtype);
  if (m == 0 || n == 0) return H3K_OK;
  if (!w8p_serves(m, n, k))
    return fail(H3K_EINVAL, "the packed-weight GEMM does not serve m=%lld n=%lld k=%lld (h3k_gemm_packed_serves)",
                (long long)m, (long long)n, (long long)k);
  if (lda < k || ldo < n) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if ((m - 1) * lda + k >= (int64_t(1) << 32)) return fail(H3K_EINVAL, "a spans 4 GiB or more (one buffer descriptor)");
  if (!a || !xs || !w8p || !s_ch || !out) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(a, 16) || lda % 16 || !aligned(w8p, 16))
    return fail(H3K_EINVAL, "int8 operands must be 16-byte aligned with 16-byte multiple row strides");
  if (!aligned(xs, 16) || !aligned(s_ch, 16) || (bias && !aligned(bias, 16)))
    return fail(H3K_EINVAL, "xs, s_ch and bias must be 16-byte aligned");
  gemm_w8p_launch(a, lda, xs, w8p, s_ch, bias, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), mode, out,
                  out_dtype, ldo, acc_out, nullptr, static_cast<hipStream_t>(stream));
  return check_launch("gemm_a8w8_packed");
}

extern "C" int64_t h3k_gemm_packed_split_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || !w8p_runs(m, n, k)) return 0;
  return w8p_split_bytes(m, n, k);
}

extern "C" int h3k_gemm_a8w8_packed_ws(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p,
                                       const float* s_ch, const void* bias, int64_t m, int64_t n, int64_t k, int mode,
                                       void* out, int out_dtype, int64_t ldo, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  if (m < 0 || n < 0 || k < 0) return fail(H3K_EINVAL, "bad GEMM shape");
  if (mode != H3K_MODE_CK && mode != H3K_MODE_EAGER) return fail(H3K_EINVAL, "mode must be ck (0) or eager (1)");
  if (out_dtype != H3K_BF16 && out_dtype != H3K_F16 && out_dtype != H3K_F32)
    return fail(H3K_EINVAL, "out dtype code %d unsupported", out_dtype);
  if (m == 0 || n == 0) return H3K_OK;
  if (!w8p_runs(m, n, k))
    return fail(H3K_EINVAL, "the packed-weight GEMM needs k a multiple of 256 (>= 512), m >= 4 and n a multiple of 4: "
                "m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (lda < k || ldo < n) return fail(H3K_EINVAL, "row strides smaller than the rows");
  if ((m - 1) * lda + k >= (int64_t(1) << 32)) return fail(H3K_EINVAL, "a spans 4 GiB or more (one buffer descriptor)");
  if (!a || !xs || !w8p || !s_ch || !out) return fail(H3K_EINVAL, "NULL pointer");
  if (!aligned(a, 16) || lda % 16 || !aligned(w8p, 16))
    return fail(H3K_EINVAL, "int8 operands must be 16-byte aligned with 16-byte multiple row strides");
  if (!aligned(xs, 16) || !aligned(s_ch, 16) || (bias && !aligned(bias, 16)))
    return fail(H3K_EINVAL, "xs, s_ch and bias must be 16-byte aligned");
  const int64_t need = w8p_split_bytes(m, n, k);
  int32_t* part = nullptr;
  if (need > 0 && out_dtype != H3K_F32 && static_cast<int64_t>(workspace_bytes) >= need) {  // else whole tiles only
    if (!workspace || !aligned(workspace, 256)) return fail(H3K_EINVAL, "workspace must be 256-byte aligned");
    part = static_cast<int32_t*>(workspace);
  }
  gemm_w8p_launch(a, lda, xs, w8p, s_ch, bias, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), mode, out,
                  out_dtype, ldo, nullptr, part, static_cast<hipStream_t>(stream));
  return check_launch("gemm_a8w8_packed_ws");
}
