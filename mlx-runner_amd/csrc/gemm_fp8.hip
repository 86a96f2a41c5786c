// mxfp8 prefill GEMM on the gfx950 scaled fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
//
// y[M, N] = x[M, K] @ deq(W)[N, K].T, W in mxfp8 (E4M3 bytes, one E8M0 scale per 32).
//
// The MFMA takes both operands in an 8-bit format with one E8M0 scale per row
// and 32-wide K block -- exactly the mxfp8 weight layout, consumed raw.  x is
// bf16 (8 significant bits); one E4M3 pass would keep 4 and miss the output
// tolerance, so a pre-pass splits x per 32-block into
//     x = hi * 2^(sh-127) + lo * 2^(sl-127)      (hi, lo E4M3; sh, sl E8M0)
// with the scale chosen as 2^ceil(log2(amax/448)) (no element is clamped).
// bf16's 8 bits fit in two 4-bit E4M3 significands, so the split is exact
// except for elements below ~2^-9 of their block's max.  The GEMM then issues
// two scaled MFMAs (hi, lo) per weight fragment into the same accumulator:
// the weight tile is loaded once, the MFMA work doubles.
//
// Tiling: 512 threads (8 waves, 4 x 2), block tile 256 (x rows) x 256 (W rows),
// K step 64, LDS double-buffered (rows padded to 80 bytes: conflict-free
// 16-byte fragment reads), one barrier per K step; each wave owns 64 x 128
// as 2 x 4 32x32 accumulators.
#include <type_traits>

#include "gemm_pipe.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

// ---------------------------------------------------------------- x split pre-pass

// LDS / pre-tiled operand swizzle of the pipelined GEMM: 16-byte slot p of row r
// (64 bytes of one K step) is stored at slot p ^ p_swz(r) of the row.
__host__ __device__ __forceinline__ int p_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// Scale byte of (row r, 32-block b) in the tile-major layout the pipelined GEMM
// loads: [r / 256][b / 4][r % 256][b % 4], i.e. for each 256-row tile and pair of
// 64-wide K steps, 256 contiguous dwords (one per row).  Needs K % 128 == 0.
__host__ __device__ __forceinline__ int64_t packed_scale_index(int64_t r, int b, int K) {
  return (((r >> 8) * (K >> 7) + (b >> 2)) * 256 + (r & 255)) * 4 + (b & 3);
}

// Two lanes per (row, 32-block), sixteen elements each, so every hi / lo store
// is one 16-byte slot.  PACKED: scales in the tile-major layout above and hi /
// lo pre-tiled the way the pipelined GEMM's LDS holds them: for each 256-row
// tile and 64-wide K step, one contiguous 16 KiB block of 1024 slots of 16
// bytes, slot 4 r + (p ^ p_swz(r)) holding bytes [16 p, 16 p + 16) of row r's
// step.  Otherwise row-major [rows, K] and [rows, K / 32].  One thread per
// (row, half block): rows * K / 16 < 2^31 (checked by the host).
//
// hi = RNE_E4M3(x / 2^sh), lo = RNE_E4M3((x - hi * 2^sh) / 2^sl) with the block
// scales sh, sl from ceil_scale_exp, so no element is clamped.  The rounding is
// v_cvt_pk_fp8_f32 (OCP E4M3, nearest-even; measured identical to a software
// nearest-even on every input this pass produces); x - hi * 2^sh is exact in f32.
// The split of 16 consecutive elements (lane pair l, l ^ 1 shares a 32-block): E4M3
// hi / lo words and the block's exponents th, tl.
__device__ __forceinline__ void split16(const uint4 q0, const uint4 q1, uint32_t (&hw)[4], uint32_t (&lw)[4], int &th,
                                        int &tl) {
  const uint32_t w8[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  float v[16];
  float amax = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    v[2 * t] = __uint_as_float(w8[t] << 16);
    v[2 * t + 1] = __uint_as_float(w8[t] & 0xFFFF0000u);
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) amax = fmaxf(amax, fabsf(v[t]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  th = amax > 0.f ? ceil_scale_exp(amax) : -127;
  // hi straight from the bf16 pairs (the conversion divides by 2^th and rounds to nearest
  // even), then back to f32 times 2^th for the residual, which is exact in f32
  const float sh = e8m0_scale_operand(th);
  float rmax = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    i16x2_t c = {0, 0};
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c, __builtin_bit_cast(bf16x2_t, w8[2 * t]), sh, false);
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c, __builtin_bit_cast(bf16x2_t, w8[2 * t + 1]), sh, true);
    hw[t] = __builtin_bit_cast(uint32_t, c);
    const f32x2_t b0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hw[t], sh, false);
    const f32x2_t b1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hw[t], sh, true);
    v[4 * t] -= b0.x;
    v[4 * t + 1] -= b0.y;
    v[4 * t + 2] -= b1.x;
    v[4 * t + 3] -= b1.y;
#pragma unroll
    for (int u = 0; u < 4; ++u) rmax = fmaxf(rmax, fabsf(v[4 * t + u]));
  }
  rmax = fmaxf(rmax, __shfl_xor(rmax, 1));
  tl = rmax > 0.f ? ceil_scale_exp(rmax) : -127;
  const float sl = e8m0_scale_operand(tl);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    i16x2_t c = {0, 0};
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(c, v[4 * t], v[4 * t + 1], sl, false);
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(c, v[4 * t + 2], v[4 * t + 3], sl, true);
    lw[t] = __builtin_bit_cast(uint32_t, c);
  }
}

// Row-major form: one thread per (row, 16 elements).
__global__ __launch_bounds__(256) void split_x_kernel(const uint16_t *__restrict__ x, uint32_t total, int rows, int K,
                                                      uint8_t *__restrict__ xh, uint8_t *__restrict__ xl,
                                                      uint8_t *__restrict__ sh, uint8_t *__restrict__ sl) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  // lanes past the end (the grid is whole blocks) compute on a clamped index and
  // store nothing; total is even, so the two lanes of a block are both live or not
  const bool live = i < total;
  const uint32_t ii = live ? i : total - 1;
  const uint32_t L = (uint32_t)K >> 4;  // threads per row
  const uint32_t r = ii / L, c = ii - r * L;
  const int b = (int)(c >> 1), j = (int)(c & 1);
  const uint4 *src = (const uint4 *)(x + (int64_t)r * K + 16 * c);
  uint32_t hw[4], lw[4];
  int th, tl;
  split16(src[0], src[1], hw, lw, th, tl);
  if (!live) return;
  const int64_t o = (int64_t)r * K + 16 * c;
  *(uint4 *)(xh + o) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  *(uint4 *)(xl + o) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  if (j == 0) {
    sh[(int64_t)r * (K >> 5) + b] = (uint8_t)(th + 127);
    sl[(int64_t)r * (K >> 5) + b] = (uint8_t)(tl + 127);
  }
}

// Pre-tiled form for the pipelined GEMM: a wave takes 16 rows x U consecutive 64-wide K
// steps; in each step lane l takes row l / 4, 16 elements l % 4 of the step, so a row's
// 64 output bytes (one slot row of the step's block) come from 4 adjacent lanes and the
// wave writes 1 KiB of consecutive slots.  All U steps' reads (16 whole 128-byte row
// pieces each) are issued before the first is split, so a wave has U x 2 KiB in flight.
// total = waves x 64 threads, waves = rows16 / 16 x S / U with S = K / 64 (S % U == 0);
// rows past `rows` (up to the 16-row group) read the last row and store nothing.
template <int U>
__global__ __launch_bounds__(256) void split_x_packed_kernel(const uint16_t *__restrict__ x, uint32_t total, int rows,
                                                             int K, uint8_t *__restrict__ xh, uint8_t *__restrict__ xl,
                                                             uint8_t *__restrict__ sh, uint8_t *__restrict__ sl) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  const bool live = i < total;  // whole waves: a wave is all live or all not
  const uint32_t ii = live ? i : total - 1;
  const uint32_t SU = ((uint32_t)K >> 6) / U, w = ii >> 6, l = ii & 63;
  const uint32_t rg = w / SU, st0 = U * (w - rg * SU);
  const uint32_t r = 16 * rg + (l >> 2);
  const uint32_t rl = (int)r < rows ? r : (uint32_t)rows - 1;
  uint4 q[U][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint4 *src = (const uint4 *)(x + (int64_t)rl * K + 16 * (4 * (st0 + u) + (l & 3)));
    q[u][0] = src[0];
    q[u][1] = src[1];
  }
  const int rr = (int)(r & 255);
  const int64_t tile = (int64_t)(r >> 8) * (K >> 6);
  const bool store = live && (int)r < rows;
  // Scale bytes: step st0 + u of row r holds blocks 2 (st0 + u) + {0, 1} (lanes l % 4 in
  // {0, 1}, {2, 3}); st0 is even, so steps u = 2P, 2P + 1 fill the four bytes of the row's
  // tile-major dword st0 / 2 + P in block order.  Each lane packs the bytes of its own
  // blocks and takes the other block's from lane l ^ 2; then lane l % 4 = 2 t + P stores
  // whole dword P of hi (t = 0) or lo (t = 1) scales.
  constexpr int PW = U / 2;
  uint32_t ph[PW], pl[PW];
#pragma unroll
  for (int p = 0; p < PW; ++p) ph[p] = pl[p] = 0u;
  const int hb = (int)((l >> 1) & 1);  // the lane's block within the step
#pragma unroll
  for (int u = 0; u < U; ++u) {
    uint32_t hw[4], lw[4];
    int th, tl;
    split16(q[u][0], q[u][1], hw, lw, th, tl);
    const uint32_t c = 4 * (st0 + u) + (l & 3);
    const int b = (int)(c >> 1), j = (int)(c & 1);
    const int sft = 8 * (2 * (u & 1) + hb);
    ph[u >> 1] |= (uint32_t)(th + 127) << sft;
    pl[u >> 1] |= (uint32_t)(tl + 127) << sft;
    if (store) {
      const int64_t o = (tile + (b >> 1)) * 16384 + 16 * (4 * rr + ((2 * (b & 1) + j) ^ p_swz(rr)));
      *(uint4 *)(xh + o) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      *(uint4 *)(xl + o) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
  }
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    ph[p] |= (uint32_t)__shfl_xor((int)ph[p], 2);
    pl[p] |= (uint32_t)__shfl_xor((int)pl[p], 2);
  }
  const int t = (int)((l >> 1) & 1), p = (int)(l & 1);
  if (store && p < PW) {
    const uint32_t v = PW == 1 ? (t ? pl[0] : ph[0]) : (t ? (p ? pl[PW - 1] : pl[0]) : (p ? ph[PW - 1] : ph[0]));
    uint8_t *dst = t ? sl : sh;
    *(uint32_t *)(dst + packed_scale_index(r, 2 * (st0 + 2 * p), K)) = v;
  }
}

// ---------------------------------------------------------------- GEMM

namespace {
constexpr int F_BM = 256, F_BN = 256, F_BK = 64, F_PITCH = 80;  // bytes per LDS row (64 + 16 pad)
constexpr int F_TILE = 256 * F_PITCH;                            // one operand tile
constexpr int F_THREADS = 512;                                   // 8 waves: 4 (M) x 2 (N)
}  // namespace

struct Fp8Smem {
  uint8_t a_hi[2][F_TILE];
  uint8_t a_lo[2][F_TILE];
  uint8_t b[2][F_TILE];
  uint8_t s_hi[2][256 * 2];
  uint8_t s_lo[2][256 * 2];
  uint8_t s_b[2][256 * 2];
};

__global__ __launch_bounds__(F_THREADS) void gemm_mxfp8_kernel(
    const uint8_t *__restrict__ xh, const uint8_t *__restrict__ xl, const uint8_t *__restrict__ sh,
    const uint8_t *__restrict__ sl, const uint8_t *__restrict__ w, const uint8_t *__restrict__ sw,
    uint16_t *__restrict__ y, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Fp8Smem &sm = *reinterpret_cast<Fp8Smem *>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave tile: rows wm*64 + [0,64), cols wn*128 + [0,128)
  int tm, tn;
  tile_of(blockIdx.x, (M + F_BM - 1) / F_BM, (N + F_BN - 1) / F_BN, &tm, &tn);
  const int m0 = tm * F_BM, n0 = tn * F_BN;
  const int nb = K >> 5;  // scale bytes per row
  const int steps = K / F_BK;

  // loader: 16-byte chunk c = tid + 512*j (j < 2) of each 256 x 64 tile: row c>>2, part c&3
  uint4 ra_h[2], ra_l[2], rb[2];
  uint16_t rs0, rs1;  // tid < 256: x-hi scales (rs0) and W scales (rs1) of row tid; else x-lo scales of row tid-256
  const int srow = tid & 255;
  const int64_t sm_row = min(m0 + srow, M - 1), sn_row = min(n0 + srow, N - 1);
  const uint8_t *s_src0 = (tid < 256 ? sh : sl) + sm_row * nb;
  const uint8_t *s_src1 = sw + sn_row * nb;

  auto gload = [&](int step) {
    const int k0 = step * F_BK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = tid + F_THREADS * j, row = c >> 2, part = c & 3;
      const int64_t mr = min(m0 + row, M - 1), nr = min(n0 + row, N - 1);
      ra_h[j] = *(const uint4 *)(xh + mr * K + k0 + part * 16);
      ra_l[j] = *(const uint4 *)(xl + mr * K + k0 + part * 16);
      rb[j] = load_stream16(w + nr * K + k0 + part * 16);
    }
    rs0 = *(const uint16_t *)(s_src0 + (k0 >> 5));
    if (tid < 256) rs1 = *(const uint16_t *)(s_src1 + (k0 >> 5));
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = tid + F_THREADS * j, row = c >> 2, part = c & 3;
      *(uint4 *)(sm.a_hi[buf] + row * F_PITCH + part * 16) = ra_h[j];
      *(uint4 *)(sm.a_lo[buf] + row * F_PITCH + part * 16) = ra_l[j];
      *(uint4 *)(sm.b[buf] + row * F_PITCH + part * 16) = rb[j];
    }
    if (tid < 256) {
      *(uint16_t *)(sm.s_hi[buf] + srow * 2) = rs0;
      *(uint16_t *)(sm.s_b[buf] + srow * 2) = rs1;
    } else {
      *(uint16_t *)(sm.s_lo[buf] + srow * 2) = rs0;
    }
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  gload(0);
  sstore(0);
  __syncthreads();
  // Operand layout of v_mfma_scale_f32_32x32x64_f8f6f4 (measured on gfx950): lane l
  // holds row l%32; its bytes 0-15 are K 16*(l/32)+[0,16) of block 0 and bytes 16-31
  // the same span of block 1 (K+32).  Its scale byte covers block l/32 of row l%32.
  const int fr = lane & 31, fh = lane >> 5, fk = fh * 16;
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) gload(s + 1);
    i32x8_t ah[2], al[2];
    int shv[2], slv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = wm * 64 + i * 32 + fr;
      const uint8_t *ph = sm.a_hi[buf] + row * F_PITCH + fk;
      const uint8_t *pl = sm.a_lo[buf] + row * F_PITCH + fk;
      const uint4 h0 = *(const uint4 *)ph, h1 = *(const uint4 *)(ph + 32);
      const uint4 l0 = *(const uint4 *)pl, l1 = *(const uint4 *)(pl + 32);
      ah[i] = i32x8_t{(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
      al[i] = i32x8_t{(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
      shv[i] = sm.s_hi[buf][row * 2 + fh];
      slv[i] = sm.s_lo[buf][row * 2 + fh];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 128 + j * 32 + fr;
      const uint8_t *p = sm.b[buf] + row * F_PITCH + fk;
      const uint4 u0 = *(const uint4 *)p, u1 = *(const uint4 *)(p + 32);
      const i32x8_t bfr = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
      const int bsc = sm.s_b[buf][row * 2 + fh];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ah[i], bfr, acc[i][j], 0, 0, 0, shv[i], 0, bsc);
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(al[i], bfr, acc[i][j], 0, 0, 0, slv[i], 0, bsc);
      }
    }
    if (s + 1 < steps) sstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: 32x32 accumulator element v of lane l is row 8*(v/4) + 4*(l/32) + v%4, col l%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (row < M && col < N) y[(int64_t)row * N + col] = f32_to_bf16_rne(acc[i][j][v]);
      }
    }
}

// ---------------------------------------------------------------- pipelined GEMM (K % 128 == 0)
//
// Same MFMA and wave layout as above (8 waves, 4 along x rows x 2 along W rows),
// in two tile sizes: TS = 256 (waves of 64 x 128) for the bulk and TS = 128
// (waves of 32 x 64) for a last partial round of the chip, split four ways so
// that it takes a quarter of a round.  The operand traffic is off the VGPRs:
//   * every operand byte goes global -> LDS directly (global_load_lds: lane i
//     of a wave writes bytes [16 i, 16 i + 16) of the wave's 1 KiB destination,
//     [4 i, 4 i + 4) for the dword form), into a 3-stage ring: the loads of step
//     s + 2 are issued while step s computes;
//   * the DMA is issued from inline assembly and waited for explicitly
//     (s_waitcnt vmcnt), so no compiler-inserted wait serialises the ring;
//   * an operand tile is TS rows x 64 bytes, unpadded; 16-byte slot p of row r is
//     stored at slot p ^ p_swz(r), so the fragment reads of 8 (or 16) consecutive
//     rows at one slot hit distinct banks; x hi / lo come pre-tiled in exactly
//     this order (a 128-row tile is one half of a 256-row block), W row-major;
//   * scales: per stage, the dword holding each row's 4 E8M0 bytes of the step
//     pair (the step uses 2 of them) for x hi, x lo and W, from the tile-major
//     copies;
//   * each wave issues exactly TS / 32 DMAs per step (3 TS / 128 tile, TS / 128
//     scale), the count the waits are written for.
namespace {
constexpr int P_BK = 64, P_STAGES = 3;
template <int TS>
struct PipeGeom {
  static constexpr int TILE = TS * P_BK;                  // one operand tile (bytes)
  static constexpr int SCALES = 4 * TS * 4;               // x hi, x lo, W scale dwords + a spare block
  static constexpr int STAGE = 3 * TILE + SCALES;         // 52 KiB at 256, 26 KiB at 128
  static constexpr size_t LDS = (size_t)P_STAGES * STAGE;
  static constexpr int TI = TS / 128;                     // tile DMAs per wave per operand
  static constexpr int IPT = TS / 64;                     // scale DMAs per scale tensor
  static constexpr int NDMA = 4 * TI;                     // DMAs per wave per step
  static constexpr int FI = TS / 128, FJ = TS / 64;       // accumulators per wave
};
}  // namespace

__device__ __forceinline__ i32x8_t p_frag(const uint8_t *base, int off) {
  const uint4 u0 = *(const uint4 *)(base + off), u1 = *(const uint4 *)(base + (off ^ 32));
  return i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
}

// Tile `bid` of the TS x TS tiling of x rows [0, M) and W rows [n_begin, n_end), over the
// K steps [s_begin, s_end).  With `part` null the tile's bf16 result goes to y; otherwise
// (a K range of a split tile) the fp32 accumulators go to `part` as they sit in the
// registers: wave w, accumulator (i, j), elements 4 v4 .. 4 v4 + 3 of lane l as the float4
// at ((w * FI * FJ + i * FJ + j) * 4 + v4) * 64 + l.
template <int TS>
__device__ __forceinline__ void pipe_tile(int bid, const uint8_t *__restrict__ xh, const uint8_t *__restrict__ xl,
                                          const uint8_t *__restrict__ sh, const uint8_t *__restrict__ sl,
                                          const uint8_t *__restrict__ w, const uint8_t *__restrict__ sw,
                                          const YOut yo, int M, int N, int K, int n_begin, int n_end,
                                          int s_begin, int s_end, float *__restrict__ part) {
  using G = PipeGeom<TS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t lds0 = lds_addr(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // wave tile: rows wm * TS / 4 + [0, TS / 4), cols wn * TS / 2 + [0, TS / 2)
  int tm, tn;
  tile_of(bid, (M + TS - 1) / TS, (n_end - n_begin + TS - 1) / TS, &tm, &tn);
  const int m0 = tm * TS, n0 = n_begin + tn * TS;
  const int steps = K / P_BK;

  // tile DMA: wave-instruction t (< TI) of this wave fills LDS slots q = (8 t + wave) * 64 + lane
  // (x hi / lo pre-tiled: a 256-row block's step is 1024 contiguous slots, rows m0 % 256 on;
  // W row-major: slot q holds row q >> 2, 16-byte part (q & 3) ^ swz(row)).  An x instruction
  // covers tile rows 16 (8 t + wave) + [0, 16); when all 16 are past the last x row (a short
  // x) it moves 4 bytes per lane instead of 16: the same instruction count (the waits count
  // them), a quarter of the bytes, and those rows' results are not stored.
  const uint8_t *ga_h[G::TI], *ga_l[G::TI], *gb[G::TI];
  bool xdead[G::TI];
#pragma unroll
  for (int t = 0; t < G::TI; ++t) {
    const int q = (8 * t + wave) * 64 + lane, row = q >> 2, part = (q & 3) ^ p_swz(row);
    const int64_t xo = (int64_t)(m0 >> 8) * steps * 16384 + ((m0 & 255) * 4 + q) * 16;
    ga_h[t] = xh + xo;
    ga_l[t] = xl + xo;
    gb[t] = w + (int64_t)min(n0 + row, N - 1) * K + part * 16;
    xdead[t] = m0 + 16 * (8 * t + wave) >= M;
  }
  // scale DMA: wave-instruction t = TI wave + h (h < TI) copies rows (t % IPT) * 64 + lane
  // of tensor t / IPT (x hi, x lo, W, all tile-major; the 4th re-reads x hi into the spare block)
  const uint8_t *gs[G::TI];
  const int pairs = K >> 7;
#pragma unroll
  for (int h = 0; h < G::TI; ++h) {
    const int t = G::TI * wave + h, tensor = t / G::IPT, row = (t % G::IPT) * 64 + lane;
    const uint8_t *src = tensor == 1 ? sl : tensor == 2 ? sw : sh;
    const int base = tensor == 2 ? n0 : m0;
    gs[h] = src + ((int64_t)(base >> 8) * pairs * 256 + (base & 255) + row) * 4;
  }
  auto issue = [&](int s) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)((s % P_STAGES) * G::STAGE);
    const int k0 = s * P_BK;
    const int64_t xs = (int64_t)s * 16384;
#pragma unroll
    for (int t = 0; t < G::TI; ++t) {
      if (xdead[t]) {
        gp_dma4(ga_h[t] + xs, st + (8 * t + wave) * 1024);
        gp_dma4(ga_l[t] + xs, st + G::TILE + (8 * t + wave) * 1024);
      } else {
        gp_dma16(ga_h[t] + xs, st + (8 * t + wave) * 1024);
        gp_dma16(ga_l[t] + xs, st + G::TILE + (8 * t + wave) * 1024);
      }
      gp_dma16(gb[t] + k0, st + 2 * G::TILE + (8 * t + wave) * 1024);
    }
    const int so = 1024 * (s >> 1);  // the step pair's block
#pragma unroll
    for (int h = 0; h < G::TI; ++h) gp_dma4(gs[h] + so, st + 3 * G::TILE + (G::TI * wave + h) * 256);
  };

  // fragment geometry (32x32x64 operand layout: lane l holds row l % 32, K bytes 16 (l / 32) + [0, 16) and +32)
  const int fr = lane & 31, fh = lane >> 5;
  int oa[G::FI], ob[G::FJ], osa[G::FI], osb[G::FJ];
#pragma unroll
  for (int i = 0; i < G::FI; ++i) {
    const int r = wm * (TS / 4) + i * 32 + fr;
    oa[i] = r * P_BK + 16 * (fh ^ p_swz(r));
    osa[i] = 3 * G::TILE + r * 4 + fh;
  }
#pragma unroll
  for (int j = 0; j < G::FJ; ++j) {
    const int r = wn * (TS / 2) + j * 32 + fr;
    ob[j] = r * P_BK + 16 * (fh ^ p_swz(r));
    osb[j] = 3 * G::TILE + 2 * TS * 4 + r * 4 + fh;
  }

  f32x16_t acc[G::FI][G::FJ];
#pragma unroll
  for (int i = 0; i < G::FI; ++i)
#pragma unroll
    for (int j = 0; j < G::FJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Ping-pong: waves 0-3 (group 0) and 4-7 (group 1) put one wave of each group on
  // every SIMD.  Barrier intervals alternate: in each, one group runs the MFMAs
  // of its step while the other issues its DMAs and reads its next fragments, so
  // the MFMA pipe of every SIMD always has a wave feeding it.  Group 0 computes
  // step k in interval 2k + 1, group 1 in 2k + 2.  DMA(k + 2) overwrites the
  // stage group 1 read in interval 2k - 1, and is issued in the loading interval
  // of step k (2k, 2k + 1); at the barrier that ends interval 2k + 1 every wave
  // waits for its DMA(k + 1) (only DMA(k + 2), NDMA loads, may remain), so stage
  // k + 1 is whole before group 0 reads it in interval 2k + 2.
  const int grp = wave >> 2;
  issue(s_begin);
  if (s_end - s_begin > 1) issue(s_begin + 1);
  if (s_end - s_begin > 1) gp_wait_barrier<G::NDMA>();
  else gp_wait_barrier<0>();

  // one step of a group: loading interval (DMAs of step s + 2 if DMA, fragments of
  // step s), barrier, computing interval, barrier.  Each call is one basic block, so
  // the scheduling barriers keep the MFMAs inside their interval.
  auto pp_step = [&](auto grp_c, auto dma_c, int s) __attribute__((always_inline)) {
    constexpr int GRP = decltype(grp_c)::value;
    constexpr bool DMA = decltype(dma_c)::value;
    if constexpr (DMA) issue(s + 2);
    const uint8_t *st = lds + (s % P_STAGES) * G::STAGE;
    const int sb = 2 * (s & 1);  // byte of the pair dword: block fh of this step
    i32x8_t ah[G::FI], al[G::FI], bf[G::FJ];
    int shv[G::FI], slv[G::FI], bsc[G::FJ];
#pragma unroll
    for (int i = 0; i < G::FI; ++i) {
      ah[i] = p_frag(st, oa[i]);
      al[i] = p_frag(st + G::TILE, oa[i]);
      shv[i] = st[osa[i] + sb];
      slv[i] = st[osa[i] + TS * 4 + sb];
    }
#pragma unroll
    for (int j = 0; j < G::FJ; ++j) {
      bf[j] = p_frag(st + 2 * G::TILE, ob[j]);
      bsc[j] = st[osb[j] + sb];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GRP == 0) gp_lds_barrier();                // ends interval 2s
    else if constexpr (DMA) gp_wait_barrier<G::NDMA>();      // ends interval 2s + 1
    else gp_wait_barrier<0>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < G::FJ; ++j)
#pragma unroll
      for (int i = 0; i < G::FI; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ah[i], bf[j], acc[i][j], 0, 0, 0, shv[i], 0, bsc[j]);
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(al[i], bf[j], acc[i][j], 0, 0, 0, slv[i], 0, bsc[j]);
      }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GRP == 1) gp_barrier_only();               // ends interval 2s + 2
    else if constexpr (DMA) gp_wait_barrier<G::NDMA>();      // ends interval 2s + 1
    else gp_wait_barrier<0>();
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
    gp_store_partial<G::FI, G::FJ>(acc, part, wave, lane, M - (m0 + wm * (TS / 4)));
    return;
  }
  (void)steps;

  // epilogue through LDS (the ring is idle: every wave has passed the last barrier,
  // after which no fragment read or DMA is outstanding); wave w's region follows w - 1's
  constexpr int REGION = 32 * G::FI * (64 * G::FJ + 32);
  static_assert(8 * REGION <= G::LDS, "the epilogue regions fit the ring");
  const bool vec = yout_vec(yo);
  gp_store_tile_bf16<G::FI, G::FJ, 0, G::FI>(acc, lds + wave * REGION, lane, yo, M, m0 + wm * (TS / 4),
                                             n0 + wn * (TS / 2), n_end, vec);
}

// Covers x rows [0, M) and W rows [n_begin, n_end) in TS x TS tiles.
template <int TS>
__global__ __launch_bounds__(F_THREADS) void gemm_mxfp8_pipe_kernel(
    const uint8_t *__restrict__ xh, const uint8_t *__restrict__ xl, const uint8_t *__restrict__ sh,
    const uint8_t *__restrict__ sl, const uint8_t *__restrict__ w, const uint8_t *__restrict__ sw,
    const YOut yo, int M, int N, int K, int n_begin, int n_end) {
  pipe_tile<TS>(blockIdx.x, xh, xl, sh, sl, w, sw, yo, M, N, K, n_begin, n_end, 0, K / P_BK, nullptr);
}

// Both tilings in one launch: blocks [0, tiles1) are the 256-tiles of W rows [0, n_split),
// the rest cover W rows [n_split, N) one of two ways:
//   * S == 0: as 128-tiles;
//   * S >= 2: as 256-tiles whose K steps are split S ways (split tiles): block tiles1 + u
//     runs K range u % S of tile u / S and leaves its fp32 accumulators in part[u] (256 KiB
//     each), which gemm_mxfp8_split_reduce_kernel then sums.
// Blocks start in index order as CUs free up, so a CU that finishes its last 256-tile
// early takes a tail block at once instead of waiting for the slowest CU at a kernel
// boundary.  (The host gives tiles1 as whole rounds, a multiple of the CU count, so on a
// CU count that is a multiple of 8 both parts keep their XCD-aware tile order; any
// tiles1 gives the same results.)
__global__ __launch_bounds__(F_THREADS) void gemm_mxfp8_pipe_split_kernel(
    const uint8_t *__restrict__ xh, const uint8_t *__restrict__ xl, const uint8_t *__restrict__ sh,
    const uint8_t *__restrict__ sl, const uint8_t *__restrict__ w, const uint8_t *__restrict__ sw,
    const YOut yo, int M, int N, int K, int n_split, int tiles1, int S, float *__restrict__ part) {
  const int b = blockIdx.x, steps = K / P_BK;
  if (b < tiles1) {
    pipe_tile<256>(b, xh, xl, sh, sl, w, sw, yo, M, N, K, 0, n_split, 0, steps, nullptr);
  } else if (S == 0) {
    pipe_tile<128>(b - tiles1, xh, xl, sh, sl, w, sw, yo, M, N, K, n_split, N, 0, steps, nullptr);
  } else {
    const int u = b - tiles1, t = u / S, k = u - t * S;
    pipe_tile<256>(t, xh, xl, sh, sl, w, sw, yo, M, N, K, n_split, N, k * steps / S, (k + 1) * steps / S,
                   part + (size_t)u * 256 * 256);
  }
}

// Every 128-tile split S ways along K, two blocks per CU (the 78 KiB ring and at most 128
// registers per lane): for x of at most 128 rows, whose 256-tiles would be mostly padding.
// Block b runs K range b % S of tile b / S into slot b of `part` (64 KiB each).
__global__ __launch_bounds__(F_THREADS, 2) void gemm_mxfp8_pipe_ksplit128_kernel(
    const uint8_t *__restrict__ xh, const uint8_t *__restrict__ xl, const uint8_t *__restrict__ sh,
    const uint8_t *__restrict__ sl, const uint8_t *__restrict__ w, const uint8_t *__restrict__ sw,
    const YOut yo, int M, int N, int K, int S, float *__restrict__ part) {
  const int b = blockIdx.x, t = b / S, k = b - t * S, steps = K / P_BK;
  pipe_tile<128>(t, xh, xl, sh, sl, w, sw, yo, M, N, K, 0, N, k * steps / S, (k + 1) * steps / S,
                 part ? part + (size_t)b * 128 * 128 : nullptr);
}

// The split tiles' results (TS-tiles of W rows [n_split, N)): one thread per float4 of a
// tile's partial layout (gp_reduce_quad), fp8_reduce_blocks<TS> blocks of 256 per tile.
template <int TS>
constexpr int fp8_reduce_blocks() {
  return 2 * PipeGeom<TS>::FI * PipeGeom<TS>::FJ * 4;
}
template <int TS>
__global__ __launch_bounds__(256) void gemm_mxfp8_split_reduce_kernel(const float *__restrict__ part,
                                                                       const YOut yo, int M, int N,
                                                                       int n_split, int S) {
  using G = PipeGeom<TS>;
  constexpr int NQ = G::FI * G::FJ * 4;  // float4s per lane per wave
  static_assert(8 * NQ * 64 == 256 * fp8_reduce_blocks<TS>(), "whole blocks per tile");
  const int g = blockIdx.x * 256 + threadIdx.x;
  const int t = g / (8 * NQ * 64), rem = g - t * (8 * NQ * 64);
  const int wave = rem / (NQ * 64), q = (rem >> 6) % NQ, lane = rem & 63;
  int tm, tn;
  tile_of(t, (M + TS - 1) / TS, (N - n_split + TS - 1) / TS, &tm, &tn);
  const int wm = wave >> 1, wn = wave & 1;
  gp_reduce_quad<G::FI, G::FJ>(part, yo, M, N, t, S, wave, q, lane, tm * TS + wm * (TS / 4),
                               n_split + tn * TS + wn * (TS / 2));
}

// K % 128: whole step pairs (the tile-major scale layout); W rows must be 16-byte
// aligned for the DMA, and the W scales 4-byte aligned for the repack.
static bool gemm_mxfp8_pipe_ok(const QmmArgs &a) {
  return a.K % 128 == 0 && (uintptr_t)a.w % 16 == 0 && (uintptr_t)a.s % 4 == 0;
}

static size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

hipError_t launch_repack_scales(const uint8_t *s, int64_t N, int nb, uint32_t *out, hipStream_t st) {
  const int dpr = nb / 4;
  const bool wide = dpr % 4 == 0 && (uintptr_t)s % 16 == 0;
  const int64_t threads = (int64_t)round256(N) * dpr / (wide ? 4 : 1);
  const int64_t blocks = (threads + 255) / 256 < 65536 ? (threads + 255) / 256 : 65536;
  if (wide)
    hipLaunchKernelGGL(repack_scales_kernel<4>, dim3(blocks), dim3(256), 0, st, s, N, nb, out);
  else
    hipLaunchKernelGGL(repack_scales_kernel<1>, dim3(blocks), dim3(256), 0, st, s, N, nb, out);
  return hipGetLastError();
}

int gemm_mxfp8_split_layout_of(const QmmArgs &a) { return gemm_mxfp8_pipe_ok(a) ? 1 : 0; }

bool gemm_mxfp8_ok(const QmmArgs &a) {
  return a.mode == MXFP8 && !a.x_f32 && a.K % F_BK == 0 && a.K > 0 && a.M > 0 && a.N > 0;
}

// Workspace: x hi, x lo (M x K bytes each), x hi / lo scales, and for the pipelined
// kernel the W scales repacked, each scale array padded to whole 256-row tiles.

// How the pipelined GEMM covers the 256-tiles of a call on `cus` CUs:
//   * a call of at most half as many tiles as CUs (short prefill chunks, narrow
//     projections) runs every tile split S ways along K (S >= 2, at most one round of
//     blocks, each at least 8 K steps): n_split = 0, tail_tiles = all tiles;
//   * otherwise whole rounds of 256-tiles over W rows [0, n_split), and when the last
//     partial round is whole W tile-columns and four times as many 128-tiles fit one
//     round, those columns [n_split, N) run as 128-tiles (S = 0);
//   * else the last round runs as it falls (n_split = N).
// (Split tiles for a last partial round of a larger call measured slower at M = 4096,
// N = 17408, K = 5120: the 64 MiB of partial sums cost more than the 128-tiles lose.)
// x of at most 128 rows runs 128-tiles instead, two blocks per CU (TS = 128): split S
// ways along K where they leave block slots idle, whole (S = 1, stored directly) where
// there are more of them than slots.
struct Fp8Plan {
  int n_split, tiles1, tail_tiles, S, TS;
};
static int fp8_split_ways(int tiles, int capacity, int steps) {
  int S = capacity / tiles;
  if (S > 8) S = 8;
  if (S > steps / 8) S = steps / 8;
  return S >= 2 ? S : 0;
}
static Fp8Plan fp8_plan(const QmmArgs &a, int cus) {
  const int tiles_m = (a.M + 255) / 256, tiles_n = (a.N + 255) / 256, steps = a.K / P_BK;
  const int T = tiles_m * tiles_n;
  Fp8Plan p{a.N, T, 0, 0, 256};
  if (cus <= 0) return p;
  const int T128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
  if (a.M <= 128) {
    const int S = fp8_split_ways(T128, 2 * cus, steps);
    return Fp8Plan{0, 0, T128, S ? S : 1, 128};
  }
  if (2 * T <= cus) {
    const int S = fp8_split_ways(T, cus, steps);
    if (S) p = Fp8Plan{0, 0, T, S, 256};
    return p;
  }
  const int rem = T % cus;
  if (rem == 0 || rem % tiles_m != 0 || 4 * rem > cus || T <= cus) return p;
  p.n_split = (tiles_n - rem / tiles_m) * 256;
  p.tiles1 = tiles_m * (tiles_n - rem / tiles_m);
  return p;
}

size_t gemm_mxfp8_workspace(const QmmArgs &a) {
  const size_t mk = round256(a.M) * a.K, nbk = (size_t)a.K / 32;
  const bool pipe = gemm_mxfp8_pipe_ok(a);
  const bool repack = pipe && !a.s_tiled;
  size_t bytes = 2 * mk + 2 * round256(a.M) * nbk + (repack ? round256(a.N) * nbk : 0);
  if (pipe) {  // the split tiles' fp32 partials, 256 KiB per block, 256-byte aligned
    const Fp8Plan p = fp8_plan(a, device_cu_count());
    if (p.S >= 2) bytes = round256(bytes) + (size_t)p.tail_tiles * p.S * p.TS * p.TS * 4;
  }
  return bytes + 256;
}

size_t tiled_scales_bytes(int64_t N, int nb) { return (size_t)round256((size_t)N) * (size_t)nb; }

int gemm_tiled_scale_bytes_per_row(const QmmArgs &a) {
  if (qmm_on_decode(a) || a.x_f32 || a.K <= 0) return 0;
  if (gemm_mxfp8_ok(a)) return gemm_mxfp8_pipe_ok(a) && (uintptr_t)a.x % 16 == 0 ? a.K / 32 : 0;
  if (gemm_nvfp4_ok(a)) return a.K / 16;
  return 0;
}

hipError_t launch_gemm_mxfp8(const QmmArgs &a, void *ws, hipStream_t st) {
  if (!gemm_mxfp8_ok(a)) return hipErrorInvalidValue;
  const size_t mk = round256(a.M) * a.K, nbk = (size_t)a.K / 32;
  uint8_t *xh = (uint8_t *)ws, *xl = xh + mk, *sh = xl + mk, *sl = sh + round256(a.M) * nbk;
  uint8_t *swp = sl + round256(a.M) * nbk;
  const bool pipe = gemm_mxfp8_pipe_ok(a);
  // one thread per (row, 16 elements); the packed form covers rows in groups of 16 and
  // U steps per thread (4 when K % 256 == 0, else 2: K % 128 == 0 there)
  const int64_t rows_t = pipe ? ((int64_t)a.M + 15) / 16 * 16 : (int64_t)a.M;
  const int U = pipe && a.K % 256 == 0 ? 4 : 2;
  const int64_t total = rows_t * (a.K / 16) / (pipe ? U : 1);
  if (rows_t * (a.K / 16) >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const unsigned sb = (unsigned)((total + 255) / 256);
  if (a.x_split_ready)
    ;  // the previous call on this stream left this x split in this workspace
  else if (pipe && U == 4)
    hipLaunchKernelGGL(split_x_packed_kernel<4>, dim3(sb), dim3(256), 0, st, (const uint16_t *)a.x, (uint32_t)total,
                       a.M, a.K, xh, xl, sh, sl);
  else if (pipe)
    hipLaunchKernelGGL(split_x_packed_kernel<2>, dim3(sb), dim3(256), 0, st, (const uint16_t *)a.x, (uint32_t)total,
                       a.M, a.K, xh, xl, sh, sl);
  else
    hipLaunchKernelGGL(split_x_kernel, dim3(sb), dim3(256), 0, st, (const uint16_t *)a.x, (uint32_t)total, a.M, a.K,
                       xh, xl, sh, sl);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int tiles = ((a.M + F_BM - 1) / F_BM) * ((a.N + F_BN - 1) / F_BN);
  if (pipe) {
    if (a.s_tiled) {
      swp = (uint8_t *)a.s_tiled;  // already tile-major
    } else {
      e = launch_repack_scales(a.s, (int64_t)a.N, a.K / 32, (uint32_t *)swp, st);
      if (e != hipSuccess) return e;
    }
    static std::atomic<uint64_t> lds256{0}, lds_split{0};
    e = ensure_dynamic_lds(lds256, (const void *)gemm_mxfp8_pipe_kernel<256>, (int)PipeGeom<256>::LDS);
    if (e == hipSuccess)
      e = ensure_dynamic_lds(lds_split, (const void *)gemm_mxfp8_pipe_split_kernel, (int)PipeGeom<256>::LDS);
    if (e != hipSuccess) return e;
    const int cus = device_cu_count();
    if (cus <= 0) return hipErrorNoDevice;
    // One block per CU at a time (the ring fills most of a CU's LDS); see fp8_plan for
    // how the last partial round runs.
    const Fp8Plan p = fp8_plan(a, cus);
    const YOut yo = yout_of(a);  // y, or a grouped call's parts
    if (p.n_split == a.N) {
      hipLaunchKernelGGL(gemm_mxfp8_pipe_kernel<256>, dim3(p.tiles1), dim3(F_THREADS), PipeGeom<256>::LDS, st, xh, xl,
                         sh, sl, a.w, swp, yo, a.M, a.N, a.K, 0, a.N);
      return hipGetLastError();
    }
    if (p.S == 0) {
      const int tiles2 = ((a.M + 127) / 128) * ((a.N - p.n_split + 127) / 128);
      hipLaunchKernelGGL(gemm_mxfp8_pipe_split_kernel, dim3(p.tiles1 + tiles2), dim3(F_THREADS), PipeGeom<256>::LDS,
                         st, xh, xl, sh, sl, a.w, swp, yo, a.M, a.N, a.K, p.n_split, p.tiles1, 0,
                         (float *)nullptr);
      return hipGetLastError();
    }
    // the partials follow the workspace's x split and (when made here) repacked scales
    const size_t part_off = round256(2 * mk + 2 * round256(a.M) * nbk + (a.s_tiled ? 0 : round256(a.N) * nbk));
    float *part = (float *)((uint8_t *)ws + part_off);
    if (p.TS == 128) {
      static std::atomic<uint64_t> lds128{0};
      e = ensure_dynamic_lds(lds128, (const void *)gemm_mxfp8_pipe_ksplit128_kernel, (int)PipeGeom<128>::LDS);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(gemm_mxfp8_pipe_ksplit128_kernel, dim3(p.tail_tiles * p.S), dim3(F_THREADS),
                         PipeGeom<128>::LDS, st, xh, xl, sh, sl, a.w, swp, yo, a.M, a.N, a.K, p.S,
                         p.S >= 2 ? part : (float *)nullptr);
      e = hipGetLastError();
      if (e != hipSuccess || p.S < 2) return e;
      hipLaunchKernelGGL(gemm_mxfp8_split_reduce_kernel<128>, dim3(p.tail_tiles * fp8_reduce_blocks<128>()), dim3(256), 0,
                         st, (const float *)part, yo, a.M, a.N, 0, p.S);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(gemm_mxfp8_pipe_split_kernel, dim3(p.tiles1 + p.tail_tiles * p.S), dim3(F_THREADS),
                       PipeGeom<256>::LDS, st, xh, xl, sh, sl, a.w, swp, yo, a.M, a.N, a.K, p.n_split,
                       p.tiles1, p.S, part);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gemm_mxfp8_split_reduce_kernel<256>, dim3(p.tail_tiles * fp8_reduce_blocks<256>()), dim3(256), 0,
                       st, (const float *)part, yo, a.M, a.N, p.n_split, p.S);
    return hipGetLastError();
  }
  if (a.parts) return hipErrorInvalidValue;  // (grouped calls run the pipelined kernels only)
  static std::atomic<uint64_t> lds_set{0};
  e = ensure_dynamic_lds(lds_set, (const void *)gemm_mxfp8_kernel, (int)sizeof(Fp8Smem));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gemm_mxfp8_kernel, dim3(tiles), dim3(F_THREADS), sizeof(Fp8Smem), st, xh, xl, sh, sl, a.w, a.s,
                     (uint16_t *)a.y, a.M, a.N, a.K);
  return hipGetLastError();
}

}  // namespace qmm
