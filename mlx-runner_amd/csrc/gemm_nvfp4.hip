// nvfp4 prefill GEMM on the bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// y[M, N] = x[M, K] @ deq(W)[N, K].T, W in nvfp4 (E2M1 nibbles, one E4M3 scale
// per 16), x bf16, fp32 accumulation, bf16 out.
//
// Why bf16 MFMA: an E2M1 value times an E4M3 scale has up to 6 significant bits,
// which no 8-bit MFMA operand format holds, and the scaled MFMAs take only
// E8M0 scales per 32; in bf16 (8 bits) the dequantized weight is exact.
//
// Same pipeline as the mxfp8 kernel: 256 x 256 block tile, K step 64, 8 waves
// in two ping-pong groups, a 3-stage LDS ring filled by LDS DMA two steps ahead,
// one barrier per interval.  The 64 elements of a step are taken in an order
// of our choosing (the same for x and W, so the sum is unchanged): K sub-step
// ks (of 4) takes elements 8 ks + [0, 8) for operand lane half 0 and
// 32 + 8 ks + [0, 8) for half 1, so a lane's four 8-element W pieces are one
// contiguous 16-byte piece of its row.  Per stage:
//   * x tile, 256 rows x 64 bf16 (128 bytes per row, moved in whole 128-byte
//     row segments); 16-byte slot S of row r stored at slot S ^ aswz(r);
//   * W tile kept in nvfp4, 256 rows x 32 bytes, row-major, moved by one
//     16-byte-per-lane DMA per wave (32 rows);
//   * the step's E4M3 scales, one dword (4 groups of 16) per W row, from the
//     tile-major repacked copy.
// Each wave owns 128 x 64 of the tile (4 x 2 accumulators).  The loading
// interval reads the wave's W fragments and scales and dequantizes them in
// registers (E2M1 -> f32, times the scale, -> bf16: exact), beside the other
// group's MFMAs; the computing interval reads x fragments per K sub-step and
// runs the MFMAs.
#include <type_traits>

#include "gemm_pipe.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {
constexpr int V_BM = 256, V_BN = 256, V_BK = 64, V_THREADS = 512;
constexpr int V_WTILE = 256 * 32;  // W: 256 rows x 64 nvfp4
constexpr int V_STILE = 1024;      // scale dwords
constexpr int V_STAGES = 3;
// Per x-tile height TM (256, or 128 for the last tile-columns of a call): the x tile,
// TM rows x 64 bf16, one stage, the ring, the x fragments per wave (FI, of 32 rows), and
// the DMAs per wave per step: FI x, 1 W, and for wave 0 the step's 256 scale dwords
// (1 KiB, one DMA).
template <int TM>
struct NvGeom {
  static constexpr int ATILE = TM * 128;
  static constexpr int STAGE = ATILE + V_WTILE + V_STILE;  // 41 KiB at 256, 25 KiB at 128
  static constexpr size_t LDS = (size_t)V_STAGES * STAGE;  // 123 KiB at 256
  static constexpr int FI = TM / 64;
  static constexpr int DMA = FI + 1, DMA_S = FI + 2;
};
// Every launch allocates the 256-row ring (the two-height kernel runs both in one launch).
constexpr size_t V_LDS = NvGeom<256>::LDS;
}  // namespace

__device__ __forceinline__ int aswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
// W tile: row r's two 16-byte halves are stored swapped when wswz(r) = 1, so that the
// fragment reads of 16 consecutive rows (one half each) fall in distinct banks (rows
// r and r + 8, and r and r + 4 on 32 banks, would otherwise share them)
__device__ __forceinline__ int wswz(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// Tile `bid` of the TM x 256 tiling of x rows [0, M) and W rows [n_begin, n_end)
// (n_begin a multiple of 256), over the K steps [s_begin, s_end).  With `part` null the
// tile's bf16 result goes to y; otherwise (a K range of a split tile) the fp32
// accumulators go to `part` (gp_store_partial's layout).
template <int TM>
__device__ __forceinline__ void nv_tile(int bid, const uint16_t *__restrict__ x, const uint8_t *__restrict__ w,
                                        const uint8_t *__restrict__ sp, const YOut yo, int M, int N, int K,
                                        int n_begin, int n_end, int s_begin, int s_end, float *__restrict__ part) {
  using G = NvGeom<TM>;
  // Wave layout: 2 (x rows) x 4 (W rows), waves of TM / 2 x 64, or at TM = 64 1 x 8, waves
  // of 64 x 32, so that each W element is dequantized by one wave of the block (at short x
  // the dequantization, not the MFMA work, is what a step costs).
  constexpr bool COLS = TM == 64;
  constexpr int XD = G::FI;                // x DMAs per wave per step
  constexpr int FI = COLS ? 2 : TM / 64;   // x fragments (32 rows) per wave
  constexpr int FJ = COLS ? 1 : 2;         // W fragments (32 rows) per wave
  constexpr int WM = COLS ? TM : TM / 2, WN = 32 * FJ;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t lds0 = lds_addr(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = COLS ? 0 : wave & 1, wn = COLS ? wave : wave >> 1;  // rows wm WM + [0, WM), cols wn WN + [0, WN)
  int tm, tn;
  tile_of(bid, (M + TM - 1) / TM, (n_end - n_begin + V_BN - 1) / V_BN, &tm, &tn);
  const int m0 = tm * TM, n0 = n_begin + tn * V_BN;
  const int steps = K / V_BK;
  const int64_t wrow = K >> 1;  // bytes per W row

  // DMA sources (step 0).  x: wave-instruction g = wave + 8 i fills slots q = 64 g + lane,
  // rows 8 g + [0, 8) of the tile.  When all 8 are past the last x row (a short x), it moves
  // 4 bytes per lane instead of 16: the same instruction count (the waits count them), a
  // quarter of the bytes, and those rows' results are not stored.
  // Every DMA source is a wave-uniform base (SGPRs: the tile's first row and the step)
  // plus a 32-bit lane offset within the tile's rows.
  const uint8_t *xb = (const uint8_t *)x + (int64_t)m0 * K * 2;
  uint32_t xoff[XD];
  bool xdead[XD];
#pragma unroll
  for (int i = 0; i < XD; ++i) {
    const int g = wave + 8 * i;
    const int q = 64 * g + lane, row = q >> 3, part = (q & 7) ^ aswz(row);
    xoff[i] = (uint32_t)((min(m0 + row, M - 1) - m0) * K + part * 8) * 2;
    xdead[i] = m0 + 8 * g >= M;
  }
  // W: wave w moves rows 32 w + lane / 2, LDS half lane % 2 of the row (the row's half
  // (lane % 2) ^ wswz(row) of the step's 32 bytes)
  const int wr = 32 * wave + (lane >> 1);
  const uint8_t *wb = w + (int64_t)n0 * wrow;
  const uint32_t woff = (uint32_t)((min(n0 + wr, N - 1) - n0) * wrow) + 16 * ((lane & 1) ^ wswz(wr));
  // scales: wave 0, lane l copies the scale dwords of rows 4 l .. 4 l + 3 (the step's 1 KiB block)
  const uint8_t *sb = sp + (int64_t)(n0 >> 8) * steps * 1024;
  const uint32_t soff = 16 * lane;
  const bool sw = wave == 0;
  auto issue = [&](int s) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)((s % V_STAGES) * G::STAGE);
#pragma unroll
    for (int i = 0; i < XD; ++i) {
      if (xdead[i]) gp_dma4s(xb + s * 128, xoff[i], st + (wave + 8 * i) * 1024);
      else gp_dma16s(xb + s * 128, xoff[i], st + (wave + 8 * i) * 1024);
    }
    gp_dma16s(wb + s * 32, woff, st + G::ATILE + wave * 1024);
    if (sw) gp_dma16s(sb + s * 1024, soff, st + G::ATILE + V_WTILE);
  };

  // fragment geometry (32x32x16 bf16 operands: lane l holds row l % 32 and, in
  // sub-step ks, the step's elements 32 fh + 8 ks + [0, 8) with fh = l / 32:
  // x slot 4 fh + ks, W dword 4 fh + ks)
  const int fr = lane & 31, fh = lane >> 5;
  // (32 rows apart, fragments differ by whole 16-row swizzle periods, so one lane offset
  // per sub-step serves every fragment: x fragment i of sub-step ks at xo[ks] + 4096 i, W
  // fragment j at ob + 1024 j, its scale dword at os + 128 j)
  const int ra = wm * WM + fr, rb = wn * WN + fr;
  const int ab = (4 * fh) ^ aswz(ra);  // physical slot of logical slot 4 fh + ks is ks ^ ab
  int xo[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) xo[ks] = ra * 128 + 16 * (ks ^ ab);
  const int ob = G::ATILE + rb * 32 + 16 * (fh ^ wswz(rb));
  const int os = G::ATILE + V_WTILE + rb * 4;

  f32x16_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Ping-pong (as in the mxfp8 kernel): group 0 (waves 0-3) loads step k in interval 2k
  // and computes it in 2k + 1, group 1 (waves 4-7) one interval later; each SIMD holds one
  // wave of each group.
  //   * Loading interval: every LDS read of the step (the W fragments and scales, and the
  //     x fragments of all four sub-steps), then the DMAs of step k + 2, then the
  //     dequantization of sub-step 0.  Stage k is therefore last read in interval 2k + 1,
  //     and DMA(k + 2), which refills stage k - 1, can be issued by each group in its
  //     loading interval of step k (2k, 2k + 1); at the barrier ending interval 2k + 1
  //     every wave waits for its DMA(k + 1) (only DMA(k + 2), DMA_S / DMA loads, remain).
  //   * Computing interval: the 32 MFMAs (8 per sub-step), with the dequantization of
  //     sub-steps 1-3 interleaved, four VALU instructions after each MFMA.  The VALU work
  //     runs beside the wave's own MFMAs, and both intervals of a SIMD carry some of it.
  //     (Measured at lm_head prefill against other splits: all four sub-steps dequantized
  //     in the loading interval 4.3% slower, two of them 1-2% slower; 3 or 2 VALU per
  //     MFMA 5-8% slower; the DMAs issued before the LDS reads within 1%, after the
  //     dequantization 5% slower.)
  const int grp = wave >> 2;
  issue(s_begin);
  if (s_end - s_begin > 1) issue(s_begin + 1);
  if (s_end - s_begin <= 1) gp_wait_barrier<0>();
  else if (sw) gp_wait_barrier<G::DMA_S>();
  else gp_wait_barrier<G::DMA>();

  auto pp_step = [&](auto grp_c, auto dma_c, int s) __attribute__((always_inline)) {
    constexpr int GRP = decltype(grp_c)::value;
    constexpr bool DMA = decltype(dma_c)::value;
    const uint8_t *st = lds + (s % V_STAGES) * G::STAGE;
    uint4 wq[FJ];
    uint32_t wsc[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      wq[j] = *(const uint4 *)(st + ob + 1024 * j);
      wsc[j] = *(const uint32_t *)(st + os + 128 * j);
    }
    bf16x8_t af[4][FI];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < FI; ++i) af[ks][i] = *(const bf16x8_t *)(st + xo[ks] + 4096 * i);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DMA) issue(s + 2);
    // W sub-step ks, fragment j: 8 nvfp4 elements times the E4M3 scale of group 2 fh + ks / 2
    bf16x8_t bf[4][FJ];
    auto deq = [&](int ks, int j) __attribute__((always_inline)) {
      const uint32_t word = ks == 0 ? wq[j].x : ks == 1 ? wq[j].y : ks == 2 ? wq[j].z : wq[j].w;
      bf[ks][j] = deq8_nvfp4(word, (wsc[j] >> (8 * (2 * fh + (ks >> 1)))) & 0xFF);
    };
#pragma unroll
    for (int j = 0; j < FJ; ++j) deq(0, j);
    // sub-step 0's W is pinned here, so that its VALU work stays in the loading interval
#pragma unroll
    for (int j = 0; j < FJ; ++j) asm volatile("" : "+v"(bf[0][j]));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GRP == 0) gp_lds_barrier();  // ends interval 2s
    else if constexpr (DMA) {                  // ends interval 2s + 1
      if (sw) gp_wait_barrier<G::DMA_S>();
      else gp_wait_barrier<G::DMA>();
    } else {
      gp_wait_barrier<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < 3) {
#pragma unroll
        for (int j = 0; j < FJ; ++j) deq(ks + 1, j);
      }
#pragma unroll
      for (int j = 0; j < FJ; ++j)
#pragma unroll
        for (int i = 0; i < FI; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], bf[ks][j], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < 4 * FI * FJ; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then four VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GRP == 1) gp_barrier_only();  // ends interval 2s + 2 (no LDS read in it)
    else if constexpr (DMA) {                   // ends interval 2s + 1
      if (sw) gp_wait_barrier<G::DMA_S>();
      else gp_wait_barrier<G::DMA>();
    } else {
      gp_wait_barrier<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto pp_run = [&](auto grp_c) __attribute__((always_inline)) {
    constexpr int GRP = decltype(grp_c)::value;
    if constexpr (GRP == 1) gp_barrier_only();  // group 1 starts one interval late
    int s = s_begin;
    for (; s + 2 < s_end; ++s) pp_step(grp_c, std::true_type{}, s);
    for (; s < s_end; ++s) pp_step(grp_c, std::false_type{}, s);
    if constexpr (GRP == 0) gp_barrier_only();  // matches group 1's extra barrier
  };
  if (grp == 0) pp_run(std::integral_constant<int, 0>{});
  else pp_run(std::integral_constant<int, 1>{});
  if (part) {  // a K range of a split tile: the raw accumulators
    gp_store_partial<FI, FJ>(acc, part, wave, lane, M - (m0 + wm * WM));
    return;
  }
  (void)steps;

  // epilogue through LDS (the ring is idle: every wave has passed the last barrier, after
  // which no fragment read or DMA is outstanding), in two halves of the wave's 128 rows
  // so that the eight regions fit the ring
  constexpr int NI = FI < 2 ? FI : 2;  // accumulator rows per half
  constexpr int REGION = 32 * NI * (64 * FJ + 32);
  // (the 256- and 128-row instances run with the 256-row ring, the 64-row one with its own)
  static_assert(8 * REGION <= (TM == 64 ? G::LDS : V_LDS), "the epilogue regions fit the launch's ring");
  const bool vec = yout_vec(yo);
  uint8_t *region = lds + wave * REGION;
  gp_store_tile_bf16<FI, FJ, 0, NI>(acc, region, lane, yo, M, m0 + wm * WM, n0 + wn * WN, n_end, vec);
  if constexpr (FI == 4)
    gp_store_tile_bf16<FI, FJ, 2, 2>(acc, region, lane, yo, M, m0 + wm * WM, n0 + wn * WN, n_end, vec);
}

__global__ __launch_bounds__(V_THREADS) void gemm_nvfp4_pipe_kernel(const uint16_t *__restrict__ x,
                                                                    const uint8_t *__restrict__ w,
                                                                    const uint8_t *__restrict__ sp,
                                                                    const YOut yo, int M, int N, int K) {
  nv_tile<256>(blockIdx.x, x, w, sp, yo, M, N, K, 0, N, 0, K / V_BK, nullptr);
}

// Every TM x 256 tile split S ways along K: block b runs K range b % S of tile b / S and
// leaves its fp32 accumulators in slot b of `part` (TM KiB each); gemm_nvfp4_split_reduce
// then sums them.  For calls of fewer tiles than CUs (short prefill chunks, narrow
// projections), which would otherwise leave most CUs idle.  The 64-row instance (x of at
// most 64 rows) moves 17 KiB per K step and runs two blocks per CU (its 51 KiB ring and
// at most 128 registers per lane), so a CU keeps two blocks' loads in flight.
template <int TM>
__device__ __forceinline__ void nv_ksplit_block(const uint16_t *__restrict__ x, const uint8_t *__restrict__ w,
                                                const uint8_t *__restrict__ sp, const YOut yo, int M,
                                                int N, int K, int S, float *__restrict__ part) {
  const int b = blockIdx.x, t = b / S, k = b - t * S, steps = K / V_BK;
  nv_tile<TM>(t, x, w, sp, yo, M, N, K, 0, N, k * steps / S, (k + 1) * steps / S,
              part ? part + (size_t)b * TM * 256 : nullptr);
}
template <int TM>
__global__ __launch_bounds__(V_THREADS) void gemm_nvfp4_pipe_ksplit_kernel(const uint16_t *__restrict__ x,
                                                                           const uint8_t *__restrict__ w,
                                                                           const uint8_t *__restrict__ sp,
                                                                           const YOut yo, int M, int N,
                                                                           int K, int S, float *__restrict__ part) {
  nv_ksplit_block<TM>(x, w, sp, yo, M, N, K, S, part);
}
__global__ __launch_bounds__(V_THREADS, 2) void gemm_nvfp4_pipe_ksplit64_kernel(const uint16_t *__restrict__ x,
                                                                                const uint8_t *__restrict__ w,
                                                                                const uint8_t *__restrict__ sp,
                                                                                const YOut yo, int M,
                                                                                int N, int K, int S,
                                                                                float *__restrict__ part) {
  nv_ksplit_block<64>(x, w, sp, yo, M, N, K, S, part);
}

// The split tiles' results: one thread per float4 of a tile's partial layout
// (gp_reduce_quad), 8 * FI * FJ * 4 * 64 threads per tile, nv_reduce_blocks<TM> blocks of 256.
template <int TM>
constexpr int nv_reduce_blocks() {
  return TM == 64 ? 2 * 2 * 1 * 4 : 2 * (TM / 64) * 2 * 4;  // 2 * FI * FJ * 4
}
template <int TM>
__global__ __launch_bounds__(256) void gemm_nvfp4_split_reduce_kernel(const float *__restrict__ part,
                                                                       const YOut yo, int M, int N, int S) {
  // the wave layout of nv_tile<TM>
  constexpr bool COLS = TM == 64;
  constexpr int FI = COLS ? 2 : TM / 64, FJ = COLS ? 1 : 2;
  constexpr int WM = COLS ? TM : TM / 2, WN = 32 * FJ;
  constexpr int NQ = FI * FJ * 4;  // float4s per lane per wave
  static_assert(8 * NQ * 64 == 256 * nv_reduce_blocks<TM>(), "whole blocks per tile");
  const int g = blockIdx.x * 256 + threadIdx.x;
  const int t = g / (8 * NQ * 64), rem = g - t * (8 * NQ * 64);
  const int wave = rem / (NQ * 64), q = (rem >> 6) % NQ, lane = rem & 63;
  int tm, tn;
  tile_of(t, (M + TM - 1) / TM, (N + V_BN - 1) / V_BN, &tm, &tn);
  const int wm = COLS ? 0 : wave & 1, wn = COLS ? wave : wave >> 1;
  gp_reduce_quad<FI, FJ>(part, yo, M, N, t, S, wave, q, lane, tm * TM + wm * WM, tn * V_BN + wn * WN);
}

// Both tile heights in one launch: blocks [0, tiles1) are the 256-row tiles of W rows
// [0, n_split), the rest the 128-row tiles of W rows [n_split, N).  Blocks start in
// index order as CUs free up, so a partial last round of 256-row tiles runs as twice as
// many half tiles, each moving 25 of the 41 KiB a full tile moves per K step.
__global__ __launch_bounds__(V_THREADS) void gemm_nvfp4_pipe_split_kernel(const uint16_t *__restrict__ x,
                                                                          const uint8_t *__restrict__ w,
                                                                          const uint8_t *__restrict__ sp,
                                                                          const YOut yo, int M, int N,
                                                                          int K, int n_split, int tiles1) {
  const int b = blockIdx.x, steps = K / V_BK;
  if (b < tiles1)
    nv_tile<256>(b, x, w, sp, yo, M, N, K, 0, n_split, 0, steps, nullptr);
  else
    nv_tile<128>(b - tiles1, x, w, sp, yo, M, N, K, n_split, N, 0, steps, nullptr);
}

static size_t round256v(size_t v) { return (v + 255) & ~(size_t)255; }

// K % 64 (whole steps; the scale dword of a step is 4 groups); x and W rows
// 16-byte aligned for the DMA, scale rows 4-byte aligned for the repack.
bool gemm_nvfp4_ok(const QmmArgs &a) {
  return a.mode == NVFP4 && !a.x_f32 && a.K % V_BK == 0 && a.K > 0 && a.M > 0 && a.N > 0 &&
         (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.w % 16 == 0 && (uintptr_t)a.s % 4 == 0;
}

// x of at most 128 rows runs its own tile height, 64 rows (two blocks per CU) up to 64
// rows and 128 up to 128, split S ways along K where the tiles leave block slots idle (at
// most one round of blocks, each at least 8 K steps) and whole (S = 1, stored directly)
// where there are more tiles than slots.  Taller x runs 256-row tiles, split the same way
// when a call has at most half as many tiles as CUs: the plan, or S = 0 for the
// whole-tile paths.
struct NvSplit {
  int TM, tiles, S;
};
static NvSplit nv_split_plan(const QmmArgs &a, int cus) {
  const int TM = a.M <= 64 ? 64 : a.M <= 128 ? 128 : 256;
  const int T = ((a.M + TM - 1) / TM) * ((a.N + V_BN - 1) / V_BN), steps = a.K / V_BK;
  if (cus <= 0 || (TM == 256 && 2 * T > cus)) return NvSplit{TM, T, 0};
  int S = (TM == 64 ? 2 * cus : cus) / T;
  if (S > 8) S = 8;
  if (S > steps / 8) S = steps / 8;
  if (S >= 2) return NvSplit{TM, T, S};
  return NvSplit{TM, T, TM == 256 ? 0 : 1};
}

// Workspace: the scales repacked tile-major, unless they come so (a.s_tiled), then (split
// tiles) the fp32 partial sums, TM KiB per block, 256-byte aligned.
size_t gemm_nvfp4_workspace(const QmmArgs &a) {
  size_t bytes = a.s_tiled ? 0 : round256v(a.N) * (size_t)(a.K / 16);
  const NvSplit p = nv_split_plan(a, device_cu_count());
  if (p.S >= 2) bytes = round256v(bytes) + (size_t)p.tiles * p.S * p.TM * 256 * 4;
  return bytes + 256;
}

hipError_t launch_gemm_nvfp4(const QmmArgs &a, void *ws, hipStream_t st) {
  if (!gemm_nvfp4_ok(a)) return hipErrorInvalidValue;
  hipError_t e = hipSuccess;
  const uint8_t *tiled = (const uint8_t *)a.s_tiled;
  if (!tiled) {
    e = launch_repack_scales(a.s, (int64_t)a.N, a.K / 16, (uint32_t *)ws, st);
    if (e != hipSuccess) return e;
    tiled = (const uint8_t *)ws;
  }
  static std::atomic<uint64_t> lds_set{0}, lds_split{0}, lds_k256{0}, lds_k128{0}, lds_k64{0};
  e = ensure_dynamic_lds(lds_set, (const void *)gemm_nvfp4_pipe_kernel, (int)V_LDS);
  if (e == hipSuccess) e = ensure_dynamic_lds(lds_split, (const void *)gemm_nvfp4_pipe_split_kernel, (int)V_LDS);
  if (e == hipSuccess) e = ensure_dynamic_lds(lds_k256, (const void *)gemm_nvfp4_pipe_ksplit_kernel<256>, (int)V_LDS);
  if (e == hipSuccess) e = ensure_dynamic_lds(lds_k128, (const void *)gemm_nvfp4_pipe_ksplit_kernel<128>, (int)V_LDS);
  if (e == hipSuccess)
    e = ensure_dynamic_lds(lds_k64, (const void *)gemm_nvfp4_pipe_ksplit64_kernel, (int)NvGeom<64>::LDS);
  if (e != hipSuccess) return e;
  const YOut yo = yout_of(a);  // y, or a grouped call's parts
  const NvSplit sp = nv_split_plan(a, device_cu_count());
  if (sp.S) {
    // (S = 1: whole tiles of this height, stored directly: no partial sums, no reduce)
    float *part = sp.S >= 2 ? (float *)((uint8_t *)ws + round256v(a.s_tiled ? 0 : round256v(a.N) * (size_t)(a.K / 16)))
                            : nullptr;
    const int blocks = sp.tiles * sp.S;
    if (sp.TM == 64) {
      hipLaunchKernelGGL(gemm_nvfp4_pipe_ksplit64_kernel, dim3(blocks), dim3(V_THREADS), NvGeom<64>::LDS, st,
                         (const uint16_t *)a.x, a.w, tiled, yo, a.M, a.N, a.K, sp.S, part);
      e = hipGetLastError();
      if (e == hipSuccess && part)
        hipLaunchKernelGGL(gemm_nvfp4_split_reduce_kernel<64>, dim3(sp.tiles * nv_reduce_blocks<64>()), dim3(256), 0,
                           st, (const float *)part, yo, a.M, a.N, sp.S);
    } else if (sp.TM == 128) {
      hipLaunchKernelGGL(gemm_nvfp4_pipe_ksplit_kernel<128>, dim3(blocks), dim3(V_THREADS), V_LDS, st,
                         (const uint16_t *)a.x, a.w, tiled, yo, a.M, a.N, a.K, sp.S, part);
      e = hipGetLastError();
      if (e == hipSuccess && part)
        hipLaunchKernelGGL(gemm_nvfp4_split_reduce_kernel<128>, dim3(sp.tiles * nv_reduce_blocks<128>()), dim3(256), 0,
                           st, (const float *)part, yo, a.M, a.N, sp.S);
    } else {
      hipLaunchKernelGGL(gemm_nvfp4_pipe_ksplit_kernel<256>, dim3(blocks), dim3(V_THREADS), V_LDS, st,
                         (const uint16_t *)a.x, a.w, tiled, yo, a.M, a.N, a.K, sp.S, part);
      e = hipGetLastError();
      if (e == hipSuccess && part)
        hipLaunchKernelGGL(gemm_nvfp4_split_reduce_kernel<256>, dim3(sp.tiles * nv_reduce_blocks<256>()), dim3(256), 0,
                           st, (const float *)part, yo, a.M, a.N, sp.S);
    }
    return e == hipSuccess ? hipGetLastError() : e;
  }
  // When the 256 x 256 tiles leave a partial last round of whole tile-columns that half
  // the CUs or fewer would run, those columns run as 128 x 256 tiles in the same launch.
  const int tiles_m = (a.M + V_BM - 1) / V_BM, tiles_n = (a.N + V_BN - 1) / V_BN;
  const int cus = device_cu_count();
  const int rem = cus > 0 ? (tiles_m * tiles_n) % cus : 0;
  int n_split = a.N;
  if (rem != 0 && rem % tiles_m == 0 && 2 * rem <= cus && tiles_m * tiles_n > cus)
    n_split = (tiles_n - rem / tiles_m) * V_BN;
  const int tiles1 = tiles_m * ((n_split + V_BN - 1) / V_BN);
  if (n_split == a.N) {
    hipLaunchKernelGGL(gemm_nvfp4_pipe_kernel, dim3(tiles1), dim3(V_THREADS), V_LDS, st, (const uint16_t *)a.x, a.w,
                       tiled, yo, a.M, a.N, a.K);
    return hipGetLastError();
  }
  const int tiles2 = ((a.M + 127) / 128) * ((a.N - n_split + V_BN - 1) / V_BN);
  hipLaunchKernelGGL(gemm_nvfp4_pipe_split_kernel, dim3(tiles1 + tiles2), dim3(V_THREADS), V_LDS, st,
                     (const uint16_t *)a.x, a.w, tiled, yo, a.M, a.N, a.K, n_split, tiles1);
  return hipGetLastError();
}

}  // namespace qmm
