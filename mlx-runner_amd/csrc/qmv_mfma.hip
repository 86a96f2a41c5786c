// Decode GEMV on the gfx950 scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4, and
// the 32x32x64 form for nvfp4 at M = 3-8): y[m, n] = sum_k x[m, k] * deq(W)[n, k]
// for x of a few rows (mxfp8 up to 16), bf16 x, K = 5120, 6144, 10240 or 17408.  nvfp4
// x of 5-16 rows at K = 5120 / 6144 runs a dequantizing kernel on the bf16 MFMA
// (qmv_deq16_kernel, below).
//
// The shapes are mlx-runner's per-token qmm calls (src/model.zig:906-908
// gate/up and :912 down, :929-944 q/k/v, :1066-1074, :1309 lm_head; M = 1
// decode, 2-4 MTP verify).  They are HBM-bound.  This path moves the
// per-element decode work off the VALU so that it no longer competes with the
// weight stream:
//
//   * W is the MFMA's B operand in its stored form: E2M1 nibbles (nvfp4) or
//     E4M3 bytes (mxfp8), never unpacked.  Lane (n, h) of the 16x16x128 MFMA
//     holds row n; the E2M1 operand of lane group h is logical K [32h, 32h+32),
//     the E4M3 operand bytes 0-15 / 16-31 are K 16h + [0,16) / 64 + 16h + [0,16)
//     (both measured on gfx950), so the B operands are plain byte ranges of a row.
//   * x is split into E4M3 hi + lo with a shared exponent per scale group:
//     hi = x with its mantissa cut to 3 bits, lo = x - hi.  Both are exact E4M3
//     values (4 significant bits) for every element within 2^13 of the group
//     maximum, so hi + lo = x exactly there; smaller elements round at 2^-21 of
//     the group maximum.
//   * mxfp8: W's E8M0 group scale and x's hi/lo exponents are the MFMA's own
//     block scales; columns (m, hi|lo) of x accumulate over K in the MFMA and
//     y = column hi + column lo.
//   * nvfp4: the E4M3 group scales (one per 16 elements) are not block scales
//     of the MFMA, so x is laid out block-diagonally: column (g, hi|lo) of the A
//     operand holds x only on group g of the 128-element chunk, output column
//     (g, .) is the group's partial dot product, and W's E4M3 byte scales it in
//     fp32: 5 VALU ops per 16 rows x 128 K (the unpacking GEMV needs ~36 per
//     2048 elements).
//
// Work split: one workgroup per CU owns a contiguous range of rows (N spread
// evenly, so every CU reads the same number of HBM bytes).  Wave q owns the K
// slice [512q, 512q + 512) and keeps the A operands of its 4 chunks in
// registers; the waves walk the range's 16-row blocks in step.  K = 17408
// (34 slices) is walked by 12 waves in 3 passes.  Per row block a wave loads
// its slice with contiguous loads, passes it through a private LDS tile into
// the MFMA layout, and writes 16 partial sums to LDS; the partials are summed
// over the waves in a fixed order, so the result is deterministic.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

constexpr int QF_REC = 272;  // x record of one (x row, 128-K chunk): 256 data bytes, then 16 zero bytes
// x rows the record area of a wave's tile is laid out for: 4, M up to 8 (mxfp8), and 8
// for mxfp8 x of 9-16 rows, whose records are made 8 rows at a time
constexpr int qf_rec_rows(int M) { return M > 8 ? 8 : M > 4 ? M : 4; }
constexpr int QF_FLUSH_MAX = 16;

// Keeps a value in its own register until this point.  The scale operands of
// v_mfma_scale_* are read after the instruction issues; the compiler does not
// treat them as in use by the MFMA and may rewrite the register right after
// it (measured: a later chunk's scale then applied to an earlier chunk).  Each
// MFMA's scale therefore stays live until the row block's results are read.
__device__ __forceinline__ void keep_live(int v) { asm volatile("" ::"v"(v)); }

// Workgroup barrier for LDS data only.  __syncthreads() also orders global memory,
// which on gfx950 means waiting for every load in flight (vmcnt(0)): the weight
// stream would drain at each barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// E4M3 hi/lo of 8 consecutive bf16 (one 16-byte piece).  GT lanes share a scale
// group (2: 16 elements, 4: 32 elements) and must be adjacent and all active.
template <int GT>
__device__ __forceinline__ void split8(const uint4 q, uint2 &hi, uint2 &lo, int &th, int &tl) {
  const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
  float xf[8];
  float amax = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    xf[2 * t] = __uint_as_float(wv[t] << 16);
    xf[2 * t + 1] = __uint_as_float(wv[t] & 0xFFFF0000u);
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(xf[t]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  if (GT == 4) amax = fmaxf(amax, __shfl_xor(amax, 2));
  th = amax > 0.f ? ceil_scale_exp(amax) : -127;  // amax * 2^-th <= 448
  // |lo| < 2^(e-3) for an element of exponent e <= e(amax), so lo * 2^-(th-3) < 256
  tl = th - 3 < -127 ? -127 : th - 3;
  // hi: the bf16 pairs with their mantissas cut to 3 bits (sign, exponent, top 3 bits),
  // divided by 2^th by the scaled conversion; lo = x - hi in f32 (exact), divided by 2^tl
  const float sh = e8m0_scale_operand(th), sl = e8m0_scale_operand(tl);
  uint32_t hw[2], lw[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    i16x2_t c = {0, 0};
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c, __builtin_bit_cast(bf16x2_t, wv[2 * t] & 0xFFF0FFF0u), sh, false);
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c, __builtin_bit_cast(bf16x2_t, wv[2 * t + 1] & 0xFFF0FFF0u), sh,
                                                  true);
    hw[t] = __builtin_bit_cast(uint32_t, c);
    float d[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float x = xf[4 * t + u];
      d[u] = x - __uint_as_float(__float_as_uint(x) & 0xFFF00000u);
    }
    i16x2_t e = {0, 0};
    e = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(e, d[0], d[1], sl, false);
    e = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(e, d[2], d[3], sl, true);
    lw[t] = __builtin_bit_cast(uint32_t, e);
  }
  hi = make_uint2(hw[0], hw[1]);
  lo = make_uint2(lw[0], lw[1]);
}

// x of one 512-element slice, split into E4M3 hi/lo records in a wave's LDS tile.
// Lane l holds elements [8l, 8l+8) of each x row m.  Record (m, c) of 128-element
// chunk c sits at tile + (m * 4 + c) * QF_REC and ends in 16 zero bytes; the
// exponent bytes (E8M0 codes) follow the records, 64 per x row.
//   nvfp4: group g (16 elements) of the chunk: hi at 32 g, lo at 32 g + 16;
//          exponent of (m, g, hi|lo, c) at 64 m + (2 g + hl) * 4 + c.
//   mxfp8: hi at [0, 128), lo at [128, 256) in K order; exponent of
//          (m, hi|lo, c, block) at 64 m + (4 hl + c) * 4 + block.
template <int MODE, int M, int LR = qf_rec_rows(M)>
__device__ __forceinline__ void qf_write_records(uint8_t *tile, const uint4 (&xin)[M], int lane) {
  uint8_t *ex = tile + 4 * LR * QF_REC;  // after the records of LR rows
  const int c = lane >> 4, kc = (lane & 15) * 8;  // chunk of the slice, offset in the chunk
#pragma unroll
  for (int m = 0; m < M; ++m) {
    uint2 hi, lo;
    int th, tl;
    split8<MODE == NVFP4 ? 2 : 4>(xin[m], hi, lo, th, tl);
    uint8_t *rec = tile + (m * 4 + c) * QF_REC;
    if constexpr (MODE == NVFP4) {
      const int g = kc >> 4, half = (kc >> 3) & 1;
      *(uint2 *)(rec + 32 * g + 8 * half) = hi;
      *(uint2 *)(rec + 32 * g + 16 + 8 * half) = lo;
      if (half == 0) {
        ex[m * 64 + (g * 2 + 0) * 4 + c] = (uint8_t)(th + 127);
        ex[m * 64 + (g * 2 + 1) * 4 + c] = (uint8_t)(tl + 127);
      }
    } else {
      *(uint2 *)(rec + kc) = hi;
      *(uint2 *)(rec + 128 + kc) = lo;
      if ((kc & 31) == 0) {
        ex[m * 64 + (0 * 4 + c) * 4 + (kc >> 5)] = (uint8_t)(th + 127);
        ex[m * 64 + (1 * 4 + c) * 4 + (kc >> 5)] = (uint8_t)(tl + 127);
      }
    }
  }
  if (lane < 4 * M) *(uint4 *)(tile + lane * QF_REC + 256) = make_uint4(0, 0, 0, 0);
}

// First row of workgroup b when N rows are spread over the grid: the first rrem
// workgroups take rbase + 1 rows, the others rbase (rbase = N / grid and rrem =
// N % grid, from the host).  A division here would cost every wave ~150 scalar
// instructions and a second kernel-argument round trip before its first load
// (measured: the first weight load issued 0.9 us after the wave started).
__device__ __forceinline__ int rows_begin(int b, int rbase, int rrem) { return b * rbase + (b < rrem ? b : rrem); }

// A unit is one wave's K slice (512 elements = 4 chunks of 128) of one 16-row block:
//   nvfp4: 16 rows x 256 bytes = 4 loads of 1 KiB (4 rows x 256 contiguous bytes each)
//   mxfp8: 16 rows x 512 bytes = 8 loads of 1 KiB (2 rows x 512 contiguous bytes each)
// plus its scale bytes (nvfp4 16 x 32, mxfp8 16 x 16).  Contiguous 1 KiB loads
// stream HBM well; the MFMA operand layout (16 rows x 64 bytes per instruction)
// read straight from HBM does not (measured 6.1-7.0 against 4.8-5.2 TB/s), so
// each unit passes through the wave's LDS tile to change layout.
template <int MODE, int M>
struct QfGeom {
  static constexpr int UB = MODE == NVFP4 ? 256 : 512;  // W bytes per row per unit
  static constexpr int PITCH = UB + 16;                 // tile row pitch: rows land on distinct banks
  static constexpr int LOADS = 16 * UB / 1024;          // 1 KiB loads per unit
  static constexpr int SB = MODE == NVFP4 ? 32 : 16;    // scale bytes per row per unit
  static constexpr int TILE = 16 * PITCH + 16 * SB;
  static constexpr int PREP = qf_rec_rows(M) * (4 * QF_REC + 64);  // x records (rows x 4 chunks) + exponents
  static constexpr int WAVE_LDS = TILE > PREP ? TILE : PREP;
};

template <int MODE>
constexpr size_t qf_lds_bytes(int M, int Q, int F) {
  const size_t prep = (size_t)qf_rec_rows(M) * (4 * QF_REC + 64), tile = QfGeom<MODE, 1>::TILE;
  return (size_t)Q * (tile > prep ? tile : prep) + (size_t)F * M * Q * 16 * 4;
}

// NMAT = 2 is the MLP form (src/model.zig:905-915): a unit's 16 MFMA columns
// are 8 rows of W (gate) and the same 8 rows of W2 (up), so a workgroup walks
// its output rows in blocks of 8 (as many units as one matrix of twice the
// rows), and the flush writes silu(gate) * up with the reference's bf16
// roundings from columns n and n + 8.  Each MFMA column depends on its own
// weight row only, so the per-row sums are those of two separate NMAT = 1
// launches and fused and unfused results are identical.  D: units whose
// weights are in flight.
//
// K longer than Q slices is walked in P passes: in pass p wave q owns slice
// p Q + q (a slice past K re-reads the last slice and its sums are replaced by
// zero), re-splits x for it and adds its partial sums to those of earlier
// passes; the partials of every row block stay in LDS until the last pass.
//
// S1 > 0 (one unit in flight, every workgroup two row blocks, the second of at most S1
// loads' rows: 4 per load in nvfp4, 2 in mxfp8): the row-block loop runs as two unrolled
// steps, and the second block's units make only their first S1 loads (the rest would
// re-read the range's last row for output rows that are dropped; their tile rows keep
// stale bytes, which reach only those rows).
//
// SL > 0 (one unit in flight, one pass, every workgroup the same 3 or more row blocks, the
// last of at most SL loads' rows per matrix): likewise for the last row block, with the
// loop's last two steps unrolled after it.
template <int MODE, int M, int Q, int NMAT, int D, int P, bool PARTS = false, int S1 = 0, int SL = 0>
__global__ __launch_bounds__(64 * Q) void qmv_mfma_kernel(int N, int K, int F, int rbase, int rrem,
                                                          const uint16_t *__restrict__ x,
                                                          const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ s, const uint8_t *__restrict__ w2,
                                                          const uint8_t *__restrict__ s2, const YOut yo) {
  using G = QfGeom<MODE, M>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  uint8_t *tile = lds + q * G::WAVE_LDS;
  float *part = (float *)(lds + Q * G::WAVE_LDS);  // [F][M][Q][16] partial sums
  constexpr int RB = NMAT == 2 ? 8 : 16;            // output rows per unit
  const int r_begin = rows_begin(blockIdx.x, rbase, rrem);
  const int r_end = rows_begin(blockIdx.x + 1, rbase, rrem);
  const int nrb = (r_end - r_begin + RB - 1) / RB;
  const int S = K >> 9;  // 512-element slices
  auto slice_of = [&](int p) __attribute__((always_inline)) {
    const int sl = p * Q + q;
    return sl < S ? sl : S - 1;
  };
  const int upp = nrb;                      // units per pass
  const int uppd = (upp + D - 1) / D * D;   // ... rounded up to whole buffer groups

  // 1) x of this wave's slices, all passes: lane l holds elements [8l, 8l+8) of each row m
  uint4 xr[P][M];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int m = 0; m < M; ++m) xr[p][m] = *(const uint4 *)(x + (int64_t)m * K + 512 * slice_of(p) + 8 * lane);
  // x goes out before the weights: a later x load would make the first split wait for
  // the first unit's loads too (the wait counter counts in issue order)
  __builtin_amdgcn_sched_barrier(0);

  // 2) the first unit's weights.  Load i, lane l: nvfp4 row 4i + l/16, bytes 16 (l%16);
  //    mxfp8 row 2i + l/32, bytes 16 (l%32).  Scales: lane l, row l/4, bytes (l%4) SB/4.
  constexpr int RPL = MODE == NVFP4 ? 4 : 2;  // rows per load
  constexpr int LPR = 64 / RPL;               // lanes per row
  const int64_t wrow = MODE == NVFP4 ? (K >> 1) : K, srow = MODE == NVFP4 ? (K >> 4) : (K >> 5);
  // unit row rr of row block rb (NMAT = 2: rr < 8 in W, rr >= 8 the same rows in W2)
  auto row_of = [&](int rb, int rr) __attribute__((always_inline)) {
    const int row = r_begin + RB * rb + (NMAT == 2 ? (rr & 7) : rr);
    return row < r_end ? row : r_end - 1;  // rows past the range re-read its last row (results dropped)
  };
  // unit (pass, row block r) lives in buffer r % D; units past a pass's last row
  // block load clamped rows and are not stored
  uint4 wv[D][G::LOADS];
  uint32_t sv0[D], sv1[D];
  // W addresses are 32-bit offsets from the matrix base (the host checks that a
  // matrix is under 4 GiB; fewer registers, and the loads take the base from
  // scalar registers), the scales' from this lane's base.
  struct UnitAddr {
    uint32_t wo[G::LOADS], so;  // byte offsets in W (or W2) and in the scales
  };
  const uint8_t *sbase = NMAT == 2 && lane >= 32 ? s2 : s;  // this lane's scale rows
  auto wbase = [&](int i) __attribute__((always_inline)) {
    return NMAT == 2 && RPL * i >= 8 ? w2 : w;  // a load's rows are all in one matrix
  };
  // unit (pass, rb); row blocks past the range read clamped rows (unused)
  auto unit_addr = [&](int pass, int rb) __attribute__((always_inline)) {
    const int sl = slice_of(pass);
    const int wcol = sl * G::UB + 16 * (lane % LPR), scol = sl * G::SB + (lane & 3) * (G::SB / 4);
    UnitAddr a;
#pragma unroll
    for (int i = 0; i < G::LOADS; ++i) a.wo[i] = (uint32_t)row_of(rb, RPL * i + lane / LPR) * (uint32_t)wrow + wcol;
    a.so = (uint32_t)row_of(rb, lane >> 2) * (uint32_t)srow + scol;
    return a;
  };
  static_assert(S1 == 0 || (NMAT == 1 && D == 1 && S1 < G::LOADS), "short row block");
  static_assert(SL == 0 || (D == 1 && P == 1 && !PARTS && S1 == 0 && SL < G::LOADS / NMAT), "short last row block");
  // load i of a unit whose rows are at most NL loads' worth per matrix (NL = G::LOADS: all)
  auto load_on = [](int i, int nl) { return (NMAT == 2 ? i % (G::LOADS / 2) : i) < nl; };
  using AllLoads = std::integral_constant<int, G::LOADS>;
  auto load_from = [&](const UnitAddr &a, int buf, auto nl) __attribute__((always_inline)) {
    constexpr int NL = decltype(nl)::value;
#pragma unroll
    for (int i = 0; i < G::LOADS; ++i)
      if (load_on(i, NL)) wv[buf][i] = load_stream16(wbase(i) + a.wo[i]);
    const uint8_t *sp = sbase + a.so;
    if constexpr (MODE == NVFP4) {
      const uint2 t2 = *(const uint2 *)sp;
      sv0[buf] = t2.x;
      sv1[buf] = t2.y;
    } else {
      sv0[buf] = *(const uint32_t *)sp;
      sv1[buf] = 0;
    }
  };
  load_from(unit_addr(0, 0), 0, AllLoads{});

  // 3) x split into records in this wave's tile (before it holds weights), then the
  //    A operands of the slice's 4 chunks into registers, kept for the pass.
  //    E4M3 A layout: lane group h, byte t holds logical K 64 (t/16) + 16 h + t%16.
  constexpr int LR = qf_rec_rows(M);
  uint8_t *ex = tile + 4 * LR * QF_REC;  // exponent bytes, 64 per x row
  const int h = lane >> 4, n = lane & 15;
  // A operands per chunk: nvfp4 one per x row; mxfp8 one per 8 x rows (MG column groups)
  constexpr int MG = MODE == NVFP4 ? 1 : (M + 7) / 8;
  constexpr int MA = MODE == NVFP4 ? M : MG;
  i32x8_t areg[4][MA];
  int asreg[4][MA];
  auto prep = [&](const uint4(&xin)[M]) __attribute__((always_inline)) {
    if constexpr (MODE == NVFP4) {
      qf_write_records<MODE, M>(tile, xin, lane);
      // column n = 4p + v: group g = 2p + v/2 of the chunk, hi (v even) or lo; nonzero only
      // where logical K is in group g, i.e. lane group g%4, byte half g/4
      const int pp = n >> 2, v = n & 3, g = 2 * pp + (v >> 1), hl = v & 1;
      const bool own = h == (g & 3);
      const int aoff0 = own && g < 4 ? 32 * g + 16 * hl : 256;
      const int aoff1 = own && g >= 4 ? 32 * g + 16 * hl : 256;
      const int ebase = (g * 2 + hl) * 4;  // + m*64 + c
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint8_t *rec = tile + (m * 4 + cc) * QF_REC;
          const uint4 u0 = *(const uint4 *)(rec + aoff0), u1 = *(const uint4 *)(rec + aoff1);
          areg[cc][m] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
          asreg[cc][m] = ex[m * 64 + ebase + cc];
        }
    } else {
      // column group gg holds x rows 8 gg + [0, 8): column n = 2 m + hl for row 8 gg + m
      // (the other columns are zero).  Its records are written to the tile, read into the
      // A operands, then overwritten by the next group's (a wave's LDS accesses run in
      // order, so the reads see this group's records).
      auto group = [&](auto gg_c) __attribute__((always_inline)) {
        constexpr int GG = decltype(gg_c)::value;
        constexpr int MR = M - 8 * GG < 8 ? M - 8 * GG : 8;  // rows of this group
        qf_write_records<MODE, MR, LR>(tile, *reinterpret_cast<const uint4(*)[MR]>(&xin[8 * GG]), lane);
        const int m = n >> 1, hl = n & 1;
        const bool lv = m < MR;
        const int aoff0 = lv ? 128 * hl + 16 * h : 256;
        const int aoff1 = lv ? 128 * hl + 64 + 16 * h : 256;
        const int am = lv ? m : 0;
        const int ebase = am * 64 + hl * 16 + h;  // + 4c: block h of chunk c
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const uint8_t *rec = tile + (am * 4 + cc) * QF_REC;
          const uint4 u0 = *(const uint4 *)(rec + aoff0), u1 = *(const uint4 *)(rec + aoff1);
          areg[cc][GG] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
          asreg[cc][GG] = ex[ebase + 4 * cc];
        }
      };
      group(std::integral_constant<int, 0>{});
      if constexpr (MG > 1) group(std::integral_constant<int, 1>{});
    }
  };
  prep(xr[0]);
#pragma unroll
  for (int d = 1; d < D; ++d) load_from(unit_addr(0, d), d, AllLoads{});

  // sum the waves' partials of row blocks [rb_first, rb_last] in wave order
  auto flush = [&](int rb_first, int rb_last) __attribute__((always_inline)) {
    lds_barrier();
    const int items = (rb_last - rb_first + 1) * M * RB;
    for (int t = tid; t < items; t += 64 * Q) {
      const int nn = t % RB, m = (t / RB) % M, rbi = t / (RB * M);
      // rb_first is a multiple of F: row block rb_first + rbi sits in slot rbi
      const int row = r_begin + RB * (rb_first + rbi) + nn;
      const float *pp = part + ((rbi * M + m) * Q) * 16 + nn;
      float sum[NMAT];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
        sum[mat] = 0.f;
#pragma unroll
        for (int qq = 0; qq < Q; ++qq) sum[mat] += pp[16 * qq + 8 * mat];
      }
      const float out = NMAT == 2 ? silu_mul_bf16(sum[0], sum[NMAT - 1]) : sum[0];
      if (row < r_end) {
        // (the part lookup only in the grouped instances: it costs registers in the loop)
        const uint16_t v = f32_to_bf16_rne(out);
        if constexpr (PARTS) {
          // x of one row leaves n0 unused; kept live here, its SGPR is not reused early
          // (a reuse made the first weight loads wait for the s_load of the part table)
          if constexpr (M == 1) asm volatile("" ::"s"(yo.n0));
          *yo.at(m, row) = v;
        } else
          yo.y0[(int64_t)m * N + row] = v;
      }
    }
    lds_barrier();
  };

  uint8_t *wt = tile, *st = tile + 16 * G::PITCH;
#pragma unroll
  for (int p = 0; p < P; ++p) {
   if (p > 0) prep(xr[p]);
   // units go in groups of D so that buffer indices are static; the units past
   // the last one are computed too (clamped rows): loads and MFMAs under a branch
   // make the compiler's wait counting conservative.  A do-while: every workgroup
   // has a row block, and the compiler then counts the next pass's x loads as
   // older than the unit loads (an exact wait before the split, not vmcnt(0)).
   int rbf = 0;  // rb % F, kept by a counter (no division in the loop)
   int r0 = 0;
   // (S1 > 0: the two row blocks as two unrolled steps of one do-while pass each, so that
   // r is a constant in each and so are its loads; SL > 0: the loop over all but the last
   // two row blocks, then those two as unrolled steps; otherwise one step, the loop as is)
#pragma unroll
   for (int step = 0; step < (S1 > 0 ? 2 : SL > 0 ? 3 : 1); ++step) {
   do {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int r = (S1 > 0 ? step : SL > 0 && step > 0 ? nrb - 3 + step : r0) + d, rb = r;
      // unit u: registers -> tile (the x records are no longer needed there), then refill
      // the buffer with unit u + D (past the last unit: clamped rows, unused)
#pragma unroll
      for (int i = 0; i < G::LOADS; ++i)
        if ((S1 == 0 || r == 0 || i < S1) && (SL == 0 || step < 2 || load_on(i, SL)))
          *(uint4 *)(wt + (RPL * i + lane / LPR) * G::PITCH + 16 * (lane % LPR)) = wv[d][i];
      if constexpr (MODE == NVFP4)
        *(uint2 *)(st + 8 * lane) = make_uint2(sv0[d], sv1[d]);
      else
        *(uint32_t *)(st + 4 * lane) = sv0[d];
      // unit r + D of this pass, or of the next one (a select, not a division).  After the
      // last pass's last unit: with one unit in flight nothing, so the wave ends without
      // waiting on a spare unit's loads; with two the clamped rows of this pass (one row,
      // cached), since loads under a branch would make the wait for the other buffer
      // conservative
      const bool wrap = p + 1 < P && r + D >= uppd;
      if constexpr (S1 > 0) {  // (D = 1 and two row blocks: step r is 0 or 1)
        if (r == 0)
          load_from(unit_addr(p, 1), d, std::integral_constant<int, (S1 > 0 ? S1 : 1)>{});
        else if (p + 1 < P)
          load_from(unit_addr(p + 1, 0), d, AllLoads{});
      } else if constexpr (SL > 0) {  // (D = 1, one pass; step 2 is the last unit)
        if (step == 0)
          load_from(unit_addr(p, r + 1), d, AllLoads{});
        else if (step == 1)
          load_from(unit_addr(p, r + 1), d, std::integral_constant<int, (SL > 0 ? SL : 1)>{});
      } else if (D > 1 || p + 1 < P || r + D < uppd) {
        load_from(unit_addr(wrap ? p + 1 : p, wrap ? r + D - uppd : r + D), d, AllLoads{});
      }
      const bool live = r < upp;
      // a slice past K (last pass only) re-read the last slice: its sums are dropped
      const bool real = P == 1 || p * Q + q < S;
      float *pslot = part + (rbf * M) * Q * 16;
      if constexpr (MODE == NVFP4) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          // B operand: row n, bytes [64c + 16h, +16) of the unit; scales of groups 2h, 2h+1
          const uint4 b = *(const uint4 *)(wt + n * G::PITCH + 64 * c + 16 * h);
          const i32x8_t bw = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
          const f32x2_t sc =
              __builtin_amdgcn_cvt_pk_f32_fp8((int)*(const uint16_t *)(st + n * G::SB + 8 * c + 2 * h), false);
          f32x4_t dd[M];
#pragma unroll
          for (int m = 0; m < M; ++m)
            dd[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(areg[c][m], bw, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0,
                                                                     4, 0, asreg[c][m], 0, 127);
          // lane (n, h) holds columns 4h..4h+3: groups 2h (hi, lo) and 2h+1 (hi, lo)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[m] += sc.x * (dd[m][0] + dd[m][1]) + sc.y * (dd[m][2] + dd[m][3]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float a = acc[m];
          a += __shfl_xor(a, 16);
          a += __shfl_xor(a, 32);
          if (live && h == 0) {
            float *dst = pslot + (m * Q + q) * 16 + n;
            a = real ? a : 0.f;
            *dst = p == 0 ? a : *dst + a;
          }
        }
      } else {
        f32x4_t dd[MG];
#pragma unroll
        for (int gg = 0; gg < MG; ++gg) dd[gg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        int bsc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          // E4M3 B operand: bytes 0-15 are K offsets 16h + [0,16) of the chunk, bytes 16-31
          // are 64 + 16h + [0,16); block h's scale is byte 4c + h of row n's scales
          const uint8_t *bp = wt + n * G::PITCH + 128 * c + 16 * h;
          const uint4 b0 = *(const uint4 *)bp, b1 = *(const uint4 *)(bp + 64);
          const i32x8_t bw = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
          bsc[c] = st[n * G::SB + 4 * c + h];
#pragma unroll
          for (int gg = 0; gg < MG; ++gg)
            dd[gg] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(areg[c][gg], bw, dd[gg], 0, 0, 0, asreg[c][gg], 0,
                                                                      bsc[c]);
        }
        // lane (n, h) holds columns 4h + v of group gg = (x row 8 gg + 2h + v/2, hi | lo)
#pragma unroll
        for (int gg = 0; gg < MG; ++gg)
#pragma unroll
          for (int v2 = 0; v2 < 2; ++v2) {
            const int m = 8 * gg + 2 * h + v2;
            if (live && m < M) {
              float *dst = pslot + (m * Q + q) * 16 + n;
              const float a = real ? dd[gg][2 * v2] + dd[gg][2 * v2 + 1] : 0.f;
              *dst = p == 0 ? a : *dst + a;
            }
          }
#pragma unroll
        for (int c = 0; c < 4; ++c) keep_live(bsc[c]);
      }
      // with several passes the host sets F >= nrb: one flush, after the last pass
      if (live && p == P - 1 && (rbf + 1 == F || rb + 1 == nrb)) flush(rb - rbf, rb);
      rbf = rbf + 1 == F ? 0 : rbf + 1;
    }
   } while (S1 == 0 && (SL > 0 ? step == 0 && ++r0 < nrb - 2 : (r0 += D) < uppd));
   }
  }
}

// nvfp4 at M = 3-4 (MTP verify): the 16x16x128 form needs one A operand per x
// row (16 columns = 8 groups x hi|lo), too many registers past M = 2.  The
// 32x32x64 MFMA has 32 A rows per 64-element chunk, room for 4 x rows x 4
// groups x hi|lo, so one A operand per chunk serves all rows:
//   A row i = 8 m + 2 g + hl holds x row m's hi (hl = 0) or lo part on group g
//   of the chunk and zero elsewhere.  Lane (i, h) of the E4M3 operand holds K
//   16 h + [0,16) in bytes 0-15 and 32 + 16 h + [0,16) in bytes 16-31 (measured),
//   so it carries the group's 16 bytes in one half when g = h or g = 2 + h.
//   Its block scale covers block h = K [32h, 32h+32) of row i.
//   B lane (j, h) holds E2M1 K [32 h, 32 h + 32) of weight row j: 16 bytes of it.
//   Output lane (j, h), element v: A row 8 (v / 4) + 4 h + v % 4, i.e. x row
//   m = v / 4, group 2 h + (v % 4) / 2, hi|lo = v % 2; the E4M3 scales of
//   groups 2h, 2h+1 of row j weight them in fp32.
// Units are 32 rows x one 512-element slice (8 KiB of E2M1, 8 loads of 1 KiB),
// staged through the wave's LDS tile as in qmv_mfma_kernel.  K longer than Q
// slices is walked in P passes (slice p Q + q in pass p); x of the next pass
// is loaded when a pass starts, so one pass of x is held in registers.
constexpr int Q32_PITCH = 272;                       // tile row pitch (256 bytes + 16)
constexpr int Q32_TILE = 32 * Q32_PITCH + 32 * 32;   // 32 rows of weights + their 32 scale bytes
constexpr int Q32_WAVE_LDS = Q32_TILE > 4 * 4 * QF_REC + 4 * 64 ? Q32_TILE : 4 * 4 * QF_REC + 4 * 64;

constexpr int Q32_FLUSH_MAX = 4;
constexpr size_t q32_lds_bytes(int M, int Q, int F) { return (size_t)Q * Q32_WAVE_LDS + (size_t)F * M * Q * 64 * 4; }

// NMAT = 2: the MLP form, a unit's 32 columns being 16 rows of W (gate) and the
// same 16 rows of W2 (up); the flush writes silu(gate) * up (as in qmv_mfma_kernel).
//
// LU < 8 (one row block per workgroup, at most 4 LU rows): the unit's loads of rows past
// the range, which every unit would make and whose sums are dropped, are not made (tile
// rows 4 LU .. 31 keep stale bytes, which reach only the dropped output rows).
//
// SL > 0 (one pass, every workgroup the same 2 or more row blocks, the last of at most 4 SL
// rows per matrix): the last row block's units make only the loads of its rows, and none
// follows the last unit; the loop's last two steps run unrolled after it.
template <int M, int Q, int P, int NMAT, bool PARTS = false, int LU = 8, int SL = 0>
__global__ __launch_bounds__(64 * Q) void qmv_mfma32_kernel(int N, int K, int F, int rbase, int rrem,
                                                            const uint16_t *__restrict__ x,
                                                            const uint8_t *__restrict__ w,
                                                            const uint8_t *__restrict__ s,
                                                            const uint8_t *__restrict__ w2,
                                                            const uint8_t *__restrict__ s2, const YOut yo) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  uint8_t *tile = lds + q * Q32_WAVE_LDS;
  float *part = (float *)(lds + Q * Q32_WAVE_LDS);  // [F][M][Q][2][32] partial sums (wave, lane half)
  constexpr int RB = NMAT == 2 ? 16 : 32;            // output rows per unit
  const int r_begin = rows_begin(blockIdx.x, rbase, rrem);
  const int r_end = rows_begin(blockIdx.x + 1, rbase, rrem);
  const int nrb = (r_end - r_begin + RB - 1) / RB;
  const int S = K >> 9;
  auto slice_of = [&](int p) __attribute__((always_inline)) {
    const int sl = p * Q + q;
    return sl < S ? sl : S - 1;
  };

  uint4 xr[M];
  auto load_x = [&](int p) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < M; ++m) xr[m] = *(const uint4 *)(x + (int64_t)m * K + 512 * slice_of(p) + 8 * lane);
  };
  load_x(0);

  // unit (pass, row block rb).  Load i, lane l: row 4i + l/16,
  // bytes 16 (l%16) of the slice; scales: lane l, row l/2, bytes 16 (l%2).
  const int64_t wrow = K >> 1, srow = K >> 4;
  // unit row rr of row block rb (NMAT = 2: rr < 16 in W, rr >= 16 the same rows in W2)
  auto row_of = [&](int rb, int rr) __attribute__((always_inline)) {
    const int row = r_begin + RB * rb + (NMAT == 2 ? (rr & 15) : rr);
    return row < r_end ? row : r_end - 1;  // rows past the range re-read its last row (results dropped)
  };
  uint4 wv[8], sv;
  // unit (pass, rb); row blocks past the range read clamped rows (unused).
  // W and scale addresses are 32-bit offsets (the host checks that a matrix is under 4 GiB).
  const uint8_t *sbase = NMAT == 2 && lane >= 32 ? s2 : s;  // this lane's scale rows
  static_assert(LU == 8 || (NMAT == 1 && LU >= 1 && LU < 8), "rows per unit");
  static_assert(SL == 0 || (P == 1 && LU == 8 && SL < 8 / NMAT), "short last row block");
  // load i of a unit of at most nl loads' rows per matrix
  auto load_on = [](int i, int nl) { return (NMAT == 2 ? i & 3 : i) < nl; };
  auto load_unit = [&](int pass, int rb, int nl = 8) __attribute__((always_inline)) {
    const int sl = slice_of(pass);
#pragma unroll
    for (int i = 0; i < LU; ++i) {
      if (!load_on(i, nl)) continue;
      const uint8_t *wm = NMAT == 2 && i >= 4 ? w2 : w;  // a load's rows are all in one matrix
      wv[i] = load_stream16(wm + ((uint32_t)row_of(rb, 4 * i + (lane >> 4)) * (uint32_t)wrow + sl * 256 +
                                  16 * (lane & 15)));
    }
    sv = *(const uint4 *)(sbase + ((uint32_t)row_of(rb, lane >> 1) * (uint32_t)srow + sl * 32 + 16 * (lane & 1)));
  };
  load_unit(0, 0);

  // A operands of the slice's 8 chunks (see above), from the x records: one per chunk
  static_assert(M <= 4, "x of up to 4 rows (one A operand per chunk)");
  constexpr int MG = 1;
  const int i = lane & 31, h = lane >> 5;
  const int am = i >> 3, ag = (i >> 1) & 3, ahl = i & 1;
  // A lane (i, h) is nonzero in bytes 0-15 (own0) or 16-31 (own1) or nowhere, the
  // same half for every chunk: only those 16 bytes are kept, the operand is
  // rebuilt with masks at each MFMA
  uint32_t amask0[MG], amask1[MG];
  int arec[MG], aex[MG];
  const int aoff = 32 * ag + 16 * ahl;  // in record (m, c8 / 2), + 128 for odd c8
#pragma unroll
  for (int G = 0; G < MG; ++G) {
    const bool alive = 4 * G + am < M;
    amask0[G] = alive && ag == h ? 0xFFFFFFFFu : 0u;
    amask1[G] = alive && ag == 2 + h ? 0xFFFFFFFFu : 0u;
    arec[G] = (alive ? 4 * G + am : 0) * 4;
    aex[G] = 4 * qf_rec_rows(M) * QF_REC + (alive ? 4 * G + am : 0) * 64 + (ag * 2 + ahl) * 4;
  }
  uint4 areg[8][MG];
  int asreg[8][MG];
  auto prep = [&]() __attribute__((always_inline)) {
    qf_write_records<NVFP4, M>(tile, xr, lane);
#pragma unroll
    for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
      for (int G = 0; G < MG; ++G) {
        // 64-element chunk c8 = half c8 % 2 of 128-element record c8 / 2: groups 4 (c8 % 2) + [0, 4)
        areg[c8][G] = *(const uint4 *)(tile + (arec[G] + (c8 >> 1)) * QF_REC + 128 * (c8 & 1) + aoff);
        asreg[c8][G] = tile[aex[G] + 4 * 8 * (c8 & 1) + (c8 >> 1)];
      }
  };

  auto flush = [&](int rb_first, int rb_last) __attribute__((always_inline)) {
    lds_barrier();
    const int items = (rb_last - rb_first + 1) * M * RB;
    for (int t = tid; t < items; t += 64 * Q) {
      const int nn = t % RB, m = (t / RB) % M, rbi = t / (RB * M);
      // rb_first is a multiple of F: row block rb_first + rbi sits in slot rbi
      const int row = r_begin + RB * (rb_first + rbi) + nn;
      const float *pp = part + ((rbi * M + m) * Q) * 64 + nn;
      float sum[NMAT];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
        sum[mat] = 0.f;
#pragma unroll
        for (int qh = 0; qh < 2 * Q; ++qh) sum[mat] += pp[32 * qh + 16 * mat];
      }
      const float out = NMAT == 2 ? silu_mul_bf16(sum[0], sum[NMAT - 1]) : sum[0];
      if (row < r_end) {
        // (the part lookup only in the grouped instances: it costs registers in the loop)
        const uint16_t v = f32_to_bf16_rne(out);
        if constexpr (PARTS)
          *yo.at(m, row) = v;
        else
          yo.y0[(int64_t)m * N + row] = v;
      }
    }
    lds_barrier();
  };

  uint8_t *wt = tile, *st = tile + 32 * Q32_PITCH;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    prep();
    if (p + 1 < P) load_x(p + 1);
    // a slice past K (last pass only) re-read the last slice: its sums are dropped
    const bool real = P == 1 || p * Q + q < S;
    // a do-while: every workgroup has a row block, and the compiler then counts the
    // next pass's x loads as older than the unit loads (exact wait before the split)
    int rb = 0, rbf = 0;  // rbf = rb % F, kept by a counter (no division in the loop)
    // (SL > 0: the units before the last two, then those two as unrolled steps)
#pragma unroll
    for (int step = 0; step < (SL > 0 ? 3 : 1); ++step) {
    do {
      if (SL > 0 && step == 0 && rb >= nrb - 2) break;
      // unit (p, rb): registers -> tile (the x records are no longer needed there), then
      // refill the registers with the next unit (past the last one: clamped, unused)
#pragma unroll
      for (int li = 0; li < LU; ++li)
        if (SL == 0 || step < 2 || load_on(li, SL))
          *(uint4 *)(wt + (4 * li + (lane >> 4)) * Q32_PITCH + 16 * (lane & 15)) = wv[li];
      *(uint4 *)(st + 16 * lane) = sv;
      // the next unit: this pass's next row block or the next pass's first; after the
      // last pass's last unit the clamped rows past the range (one row, cached), except
      // with one row block and one pass (dropped there: faster at K = 5120 / 6144, slower
      // with several passes)
      const bool wrap = p + 1 < P && rb + 1 >= nrb;
      if constexpr (SL > 0) {  // the next unit: full, or the short last one, or none
        if (step == 0)
          load_unit(p, rb + 1);
        else if (step == 1)
          load_unit(p, rb + 1, SL);
      } else if constexpr (LU < 8 && P == 1) {  // one row block and one pass: no next unit
      } else {
        load_unit(wrap ? p + 1 : p, wrap ? 0 : rb + 1);
      }
      float acc[M];
#pragma unroll
      for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
      for (int c8 = 0; c8 < 8; ++c8) {
        const uint4 b = *(const uint4 *)(wt + i * Q32_PITCH + 32 * c8 + 16 * h);
        // the MFMA of chunk c8 waits for the sums of chunk c8 - 1: issued any earlier,
        // the chunks' 16 output registers would all be live at once
        int b0 = (int)b.x;
#pragma unroll
        for (int m = 0; m < M; ++m) asm volatile("" : "+v"(b0) : "v"(acc[m]));
        const i32x8_t bw = {b0, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
        const f32x2_t sc = __builtin_amdgcn_cvt_pk_f32_fp8((int)*(const uint16_t *)(st + i * 32 + 4 * c8 + 2 * h), false);
#pragma unroll
        for (int G = 0; G < MG; ++G) {
          // (the masks pass through asm so that the masked operands are not hoisted out of
          // the loop as invariants: that would hold all 8 full operands in registers)
          uint32_t k0 = amask0[G], k1 = amask1[G];
          asm volatile("" : "+v"(k0), "+v"(k1));
          const uint4 ad = areg[c8][G];
          const i32x8_t aw = {(int)(ad.x & k0), (int)(ad.y & k0), (int)(ad.z & k0), (int)(ad.w & k0),
                              (int)(ad.x & k1), (int)(ad.y & k1), (int)(ad.z & k1), (int)(ad.w & k1)};
          const f32x16_t dd = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              aw, bw, f32x16_t{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, 0, 4,
              0, asreg[c8][G], 0, 127);
#pragma unroll
          for (int mm = 0; mm < 4; ++mm) {
            const int m = 4 * G + mm;
            if (m < M) acc[m] += sc.x * (dd[4 * mm] + dd[4 * mm + 1]) + sc.y * (dd[4 * mm + 2] + dd[4 * mm + 3]);
          }
        }
      }
      // every lane stores its half's sums (no branch: the compiler would sink the
      // accumulation of rows m > 0 into it and keep all chunks' outputs live)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float *dst = part + ((rbf * M + m) * Q + q) * 64 + lane;
        const float a = real ? acc[m] : 0.f;
        *dst = p == 0 ? a : *dst + a;
      }
#pragma unroll
      for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
        for (int G = 0; G < MG; ++G) keep_live(asreg[c8][G]);
      // with several passes the host sets F >= nrb: one flush, after the last pass
      if (p == P - 1 && (rbf + 1 == F || rb + 1 == nrb)) flush(rb - rbf, rb);
      rbf = rbf + 1 == F ? 0 : rbf + 1;
    } while (SL > 0 ? (step == 0 ? ++rb < nrb - 2 : (++rb, false)) : ++rb < nrb);
    }
  }
}


// nvfp4 x of 5-16 rows.  The scaled-MFMA forms above hold one block-diagonal A operand
// per x row (or per 4 rows): past 8 rows they run out of registers, and from 5 rows their
// MFMA and scaling work per unit grows with every row.  Here W is
// dequantized instead (E2M1 x E4M3 -> bf16, exact) and the bf16 MFMA
// (v_mfma_f32_16x16x32_bf16) takes all 16 x rows as its A rows, so the cost per unit is
// the dequantization (~2 VALU ops per weight), the same for any x of up to 16 rows.
// Work split as in qmv_mfma_kernel: one workgroup per CU owns a contiguous row range,
// wave q owns the K slice [512 q, 512 q + 512) (K = Q slices, one pass), units are 16
// rows x one slice, staged through the wave's LDS tile (1 KiB-contiguous loads).
//   The 512 elements of a slice are taken in an order chosen for the tile: MFMA c
// (of 16) gives lane group h the elements 128 h + 8 c + [0, 8), the same for x and W,
// so the sum is unchanged.  Lane (n, h) then reads W row n's bytes [64 h, 64 h + 64)
// of the unit (four 16-byte reads) and the E4M3 bytes 8 h .. 8 h + 7 of its 32 (the
// scale of MFMA c is byte c / 2), and holds x row n's elements 512 q + 128 h + [0, 128)
// as its 16 A operands for the whole call (64 registers; rows from M on are zero).
//   Output lane (n, h), element v: x row 4 h + v, W row n.  Partial sums go to LDS per
// (row block, x row, wave) and are summed over the waves in a fixed order.
constexpr int QD_PITCH = 272;                     // tile row pitch (256 bytes + 16)
constexpr int QD_TILE = 16 * QD_PITCH + 16 * 32;  // 16 rows of W + their 32 scale bytes
constexpr int QD_FLUSH_MAX = 8;
constexpr size_t qd_lds_bytes(int Q, int F) { return (size_t)Q * QD_TILE + (size_t)F * 16 * Q * 16 * 4; }

template <int Q>
__global__ __launch_bounds__(64 * Q) void qmv_deq16_kernel(int N, int K, int M, int F, int rbase, int rrem,
                                                           const uint16_t *__restrict__ x,
                                                           const uint8_t *__restrict__ w,
                                                           const uint8_t *__restrict__ s, uint16_t *__restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  uint8_t *wt = lds + q * QD_TILE, *st = wt + 16 * QD_PITCH;
  float *part = (float *)(lds + Q * QD_TILE);  // [F][16 x rows][Q][16 W rows] partial sums
  const int r_begin = rows_begin(blockIdx.x, rbase, rrem);
  const int r_end = rows_begin(blockIdx.x + 1, rbase, rrem);
  const int nrb = (r_end - r_begin + 15) / 16;
  const int n = lane & 15, h = lane >> 4;

  // 1) x: the A operands of the slice's 16 MFMAs (rows from M on: zero)
  bf16x8_t af[16];
  {
    const bool live = n < M;
    const uint4 *xp = (const uint4 *)(x + (int64_t)(live ? n : 0) * K + 512 * q + 128 * h);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      uint4 v = xp[c];
      if (!live) v = make_uint4(0, 0, 0, 0);
      af[c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2) units.  Load i (of 4), lane l: row 4 i + l / 16 of the block, bytes 16 (l % 16) of the
  //    slice's 256; scales: lane l, row l / 4, bytes 8 (l % 4) of the slice's 32.  Rows past
  //    the range re-read its last row (results dropped); W offsets are 32-bit (the host
  //    checks that the matrix is under 4 GiB).
  const uint32_t wrow = (uint32_t)(K >> 1), srow = (uint32_t)(K >> 4);
  auto row_of = [&](int rb, int rr) __attribute__((always_inline)) {
    const int row = r_begin + 16 * rb + rr;
    return (uint32_t)(row < r_end ? row : r_end - 1);
  };
  uint4 wv[4];
  uint2 sv;
  auto load_unit = [&](int rb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = load_stream16(w + row_of(rb, 4 * i + (lane >> 4)) * wrow + 256 * q + 16 * (lane & 15));
    sv = *(const uint2 *)(s + row_of(rb, lane >> 2) * srow + 32 * q + 8 * (lane & 3));
  };
  load_unit(0);

  // sum the waves' partials of row blocks [rb_first, rb_last] in wave order
  auto flush = [&](int rb_first, int rb_last) __attribute__((always_inline)) {
    lds_barrier();
    const int items = (rb_last - rb_first + 1) * M * 16;
    for (int t = tid; t < items; t += 64 * Q) {
      const int nn = t & 15, m = (t >> 4) % M, rbi = t / (16 * M);
      const int row = r_begin + 16 * (rb_first + rbi) + nn;
      const float *pp = part + ((rbi * 16 + m) * Q) * 16 + nn;
      float sum = 0.f;
#pragma unroll
      for (int qq = 0; qq < Q; ++qq) sum += pp[16 * qq];
      if (row < r_end) y[(int64_t)m * N + row] = f32_to_bf16_rne(sum);
    }
    lds_barrier();
  };

  // a do-while: every workgroup has a row block
  int rb = 0, rbf = 0;  // rbf = rb % F, kept by a counter
  do {
    // unit rb: registers -> tile, then refill them with unit rb + 1 (after the last unit
    // nothing: the wave ends without waiting on a spare unit's loads).  One wave's LDS
    // accesses run in order: the reads below see this unit.
#pragma unroll
    for (int i = 0; i < 4; ++i) *(uint4 *)(wt + (4 * i + (lane >> 4)) * QD_PITCH + 16 * (lane & 15)) = wv[i];
    *(uint2 *)(st + 8 * lane) = sv;
    if (rb + 1 < nrb) load_unit(rb + 1);
    uint4 wq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wq[i] = *(const uint4 *)(wt + n * QD_PITCH + 64 * h + 16 * i);
    const uint2 sc8 = *(const uint2 *)(st + n * 32 + 8 * h);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const uint4 &u = wq[c >> 2];
      const uint32_t word = (c & 3) == 0 ? u.x : (c & 3) == 1 ? u.y : (c & 3) == 2 ? u.z : u.w;
      const uint32_t sb = ((c >> 1) < 4 ? sc8.x >> (8 * (c >> 1)) : sc8.y >> (8 * ((c >> 1) - 4))) & 0xFF;
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[c], deq8_nvfp4(word, sb), acc, 0, 0, 0);
    }
    float *pslot = part + (rbf * 16) * Q * 16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * h + v;
      if (m < M) pslot[(m * Q + q) * 16 + n] = acc[v];
    }
    if (rbf + 1 == F || rb + 1 == nrb) flush(rb - rbf, rb);
    rbf = rbf + 1 == F ? 0 : rbf + 1;
  } while (++rb < nrb);
}
}  // namespace

// Waves per workgroup (Q) and passes (P) for K, the model's row lengths:
// K = 5120 (10 slices of 512: Q = 10, P = 1), 6144 (o_proj / out_proj: 12
// slices, Q = 12, P = 1), 10240 (mtp.fc: 20 slices, Q = 10, P = 2) and 17408
// (down: 34 slices, Q = 12, P = 3, two slices of the last pass past K).
struct QfShape {
  int Q, P;
};
static QfShape qf_shape(int K) {
  switch (K) {
    case 5120: return {10, 1};
    case 6144: return {12, 1};
    case 10240: return {10, 2};
    case 17408: return {12, 3};
    default: return {0, 0};
  }
}

static int qf_cus() { return device_cu_count(); }

// Units per workgroup: row blocks of 16 rows (8 output rows in the MLP form).
static int qf_nrb(const QmmArgs &a, int cus, int nmat = 1) {
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int rb = nmat == 2 ? 8 : 16;
  return ((a.N + grid - 1) / grid + rb - 1) / rb;
}

constexpr size_t QF_LDS_MAX = 160 * 1024;

// Row blocks per partial-sum flush: up to QF_FLUSH_MAX, as many as fit the LDS.
static int qf_flush_rows(const QmmArgs &a, int nrb) {
  const QfShape g = qf_shape(a.K);
  int F = nrb < QF_FLUSH_MAX ? nrb : QF_FLUSH_MAX;
  while (F > 1 && (a.mode == NVFP4 ? qf_lds_bytes<NVFP4>(a.M, g.Q, F) : qf_lds_bytes<MXFP8>(a.M, g.Q, F)) > QF_LDS_MAX)
    --F;
  return F;
}

static bool q32_ok(const QmmArgs &a);

// nvfp4 x of 5-16 rows on the dequantizing kernel: K of one pass (5120: Q = 10, 6144: Q = 12).
static bool qd_ok(const QmmArgs &a) {
  if (a.mode != NVFP4 || a.x_f32 || a.M < 5 || a.M > 16 || a.N < 16) return false;
  // at 5-8 rows the unpacking GEMV stays ahead on short matrices (N = 48: 5.0 against
  // 5.9 us at M = 5; N = 1024: 6.7 against 6.1)
  if (a.M <= 8 && a.N < 1024) return false;
  const QfShape g = qf_shape(a.K);
  if (g.Q == 0 || g.P != 1 || qf_cus() == 0) return false;
  if ((int64_t)a.N * (a.K / 2) >= ((int64_t)1 << 32)) return false;  // 32-bit offsets within W
  return ((((uintptr_t)a.x) | ((uintptr_t)a.w)) & 15) == 0 && ((uintptr_t)a.s & 7) == 0;
}

bool qmv_mfma_ok(const QmmArgs &a) {
  // nvfp4 x of 5-16 rows at K = 5120 / 6144: the dequantizing kernel (N = 17408, K = 5120:
  // 14.9-15.5 us at 5-8 rows against 17.1-19.3 on the 32x32x64 form, 16.0-17.9 us at 9-16
  // rows against 24.9-25.5 on the prefill GEMM's split tiles)
  if (a.mode == NVFP4 && a.M >= 5 && qd_ok(a)) return true;
  if (a.mode == NVFP4 && a.M > 8) return false;
  // (mxfp8 holds x rows as A columns (m, hi|lo): 16 columns per operand, 8 rows, and two
  // operands per chunk for 9-16 rows; nvfp4 runs 3-8 rows on the 32x32x64 form, two
  // operands per chunk from 5 rows)
  if (a.x_f32 || a.M < 1 || a.N < 16 || a.M > (a.mode == MXFP8 ? 16 : 8)) return false;
  // nvfp4 at M = 3-4 runs the 32x32x64 form (the 16x16x128 form's A operands would
  // not fit in registers); measured faster than the unpacking GEMV from N = 4096
  // (N = 5120, K = 5120, M = 3: 7.8 against 9.4 us; gate+up M = 3: 22.8 against 30.7;
  // down M = 3: 17.1 against 22.5)
  if (a.mode == NVFP4 && a.M > 2) return a.N >= 4096 && q32_ok(a);
  const QfShape g = qf_shape(a.K);
  if (g.Q == 0) return false;
  // x of every pass is held in registers: 6-8 rows fit two passes, 9-16 rows one
  if ((a.M > 5 && g.P == 3) || (a.M > 8 && g.P > 1)) return false;
  // Where this path is faster than the unpacking GEMV (measured on the 256-CU
  // MI355X): nvfp4 at M = 1 at K = 17408 (N = 5120: 11.8 against 12.4 us) and at one
  // pass from N = 4096, except with 17-24 rows per workgroup (two row blocks, the second
  // short: 5120 x 5120 4.7 against 5.3 us, 6144 x 5120 5.2 against 5.4, 5120 x 6144 5.2
  // against 5.3; 12288 x 5120 7.0 against 7.9, 10240 x 5120 6.5 against 7.1, the q+k+v
  // group of 14336 rows 8.3 against 8.9).  At M >= 2 from N = 4096.
  if (a.M == 1 && a.mode == NVFP4 && g.P == 1 && qf_cus() > 0) {
    const int rmax = (a.N + qf_cus() - 1) / qf_cus();
    if (rmax > 16 && rmax <= 24) return false;
  }
  // mxfp8 at M = 1: the unpacking GEMV at K = 5120, where it decodes at 1 VALU op per
  // weight byte and streams faster; past K = 5120 it walks the rows with its long-row
  // kernel and this path is faster (N = 5120: 7.7 against 8.1 us at K = 6144, 15.75
  // against 17.0 at K = 17408)
  if (a.M == 1 && a.mode == MXFP8 && a.K == 5120) return false;
  if (a.N < 4096) return false;
  // several passes keep every row block's partial sums in LDS
  if (g.P > 1 && (qf_cus() == 0 || qf_flush_rows(a, qf_nrb(a, qf_cus())) < qf_nrb(a, qf_cus()))) return false;
  if ((((uintptr_t)a.x) | ((uintptr_t)a.w)) & 15) return false;
  if (((uintptr_t)a.s) & 7) return false;  // scale slices are read as 8 (nvfp4) / 4 (mxfp8) bytes
  // W and scale addresses are 32-bit offsets within the matrix
  if ((int64_t)a.N * (a.mode == NVFP4 ? a.K / 2 : a.K) >= ((int64_t)1 << 32)) return false;
  return true;
}

static bool q32_mlp_ok(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up);

// The fused MLP form: the 16x16x128 kernel (nvfp4 M <= 2, mxfp8 M <= 4) and the
// 32x32x64 kernel at one pass (nvfp4 M = 3-4, K = 5120).
bool qmv_mfma_mlp_ok(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up) {
  if (!qmv_mfma_ok(a) || a.K != 5120 || a.M > 4) return false;
  if (a.mode == NVFP4 && a.M > 2) return q32_mlp_ok(a, w_up, s_up);
  return (((uintptr_t)w_up) & 15) == 0 && (((uintptr_t)s_up) & 7) == 0;
}

template <int MODE, int M, int Q, int NMAT, int D, int P, bool PARTS = false, int S1 = 0, int SL = 0>
static hipError_t launch_qf(const QmmArgs &a, const uint8_t *w2, const uint8_t *s2, int grid, int F,
                            hipStream_t st) {
  auto kern = qmv_mfma_kernel<MODE, M, Q, NMAT, D, P, PARTS, S1, SL>;
  const size_t lds = qf_lds_bytes<MODE>(M, Q, F);
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t e = ensure_dynamic_lds(lds_set, (const void *)kern, 160 * 1024);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * Q), lds, st, a.N, a.K, F, a.N / grid, a.N % grid,
                     (const uint16_t *)a.x, a.w, a.s, w2, s2, yout_of(a));
  return hipGetLastError();
}

// Loads (of RPL rows each, per matrix) of the last row block of RB-row blocks when every
// workgroup has the same min_nb or more row blocks and the last is short; 0 otherwise.
static int qf_short_last(const QmmArgs &a, int grid, int RB, int min_nb = 3, int RPL = 4) {
  const int rmin = a.N / grid, rmax = rmin + (a.N % grid ? 1 : 0);
  const int nb = (rmax + RB - 1) / RB;
  if (nb < min_nb || (rmin + RB - 1) / RB != nb) return 0;
  const int sl = (rmax - RB * (nb - 1) + RPL - 1) / RPL;
  return sl < RB / RPL ? sl : 0;
}

// One unit in flight per wave at every size.  (Two, once the rule for ranges of 1-4 row
// blocks, measured slower on the current kernels at every such shape: nvfp4 M = 2 at
// 4096 / 12288 x 5120 6.19 -> 4.79 / 9.71 -> 7.41 us with one; the second unit of a
// one-block range was a clamped re-read.)
// (grouped calls, PARTS, and the MLP form run K = 5120 only)
template <int MODE, int M, int NMAT, bool PARTS = false>
static hipError_t launch_qf_d(const QmmArgs &a, const uint8_t *w2, const uint8_t *s2, int grid, int F, int nrb,
                              hipStream_t st) {
  if constexpr (NMAT == 1 && !PARTS) {
    const QfShape g = qf_shape(a.K);
    // 17-20 rows per workgroup (5120 rows: the down projection, o_proj, out_proj): two row
    // blocks, the second's units make only the loads of its 4 rows (nvfp4 x of 2 rows at
    // 5120 x 17408: 12.71 -> 11.89 us; at one row 10.89 -> 11.0, not used there)
    const int rmin = a.N / grid, rmax = rmin + (a.N % grid ? 1 : 0);
    const bool short2 = rmin > 16 && rmax <= 20 && (MODE == MXFP8 || M == 2);
    constexpr int S1 = MODE == NVFP4 ? 1 : 2;
    if (g.P == 3) {
      if constexpr (M <= 5)
        if (short2) return launch_qf<MODE, M, 12, 1, 1, 3, false, S1>(a, w2, s2, grid, F, st);
      if constexpr (M <= 5) return launch_qf<MODE, M, 12, 1, 1, 3>(a, w2, s2, grid, F, st);
      return hipErrorInvalidValue;  // (qmv_mfma_ok: x of three passes would not fit in registers)
    }
    if (g.P == 2) {
      if constexpr (M <= 8) return launch_qf<MODE, M, 10, 1, 1, 2>(a, w2, s2, grid, F, st);
      return hipErrorInvalidValue;
    }
    if (g.Q == 12) {
      if (short2) return launch_qf<MODE, M, 12, 1, 1, 1, false, S1>(a, w2, s2, grid, F, st);
      if constexpr (MODE == NVFP4) {
        switch (qf_short_last(a, grid, 16)) {
          case 1: return launch_qf<MODE, M, 12, 1, 1, 1, false, 0, 1>(a, w2, s2, grid, F, st);
          case 2: return launch_qf<MODE, M, 12, 1, 1, 1, false, 0, 2>(a, w2, s2, grid, F, st);
          case 3: return launch_qf<MODE, M, 12, 1, 1, 1, false, 0, 3>(a, w2, s2, grid, F, st);
          default: break;
        }
      }
      return launch_qf<MODE, M, 12, 1, 1, 1>(a, w2, s2, grid, F, st);
    }
  }
  // (the MLP form and the grouped form at nvfp4 M = 2 would spill with two units in flight)
  // (nor x of 9-16 rows, whose x and A operands take twice the registers)
  // K = 5120, two row blocks of which the second has 4 or 8 rows (5120 rows: 20, 6144: 24):
  // the short second block (mxfp8 5120 x 5120: 7.80 -> 6.70 us at M = 2, 8.42 -> 7.30 at
  // M = 4, against two units in flight)
  if constexpr (NMAT == 1 && !PARTS && M <= 8 && (MODE == MXFP8 ? M >= 2 : M == 2)) {
    const int rmin = a.N / grid, rmax = rmin + (a.N % grid ? 1 : 0);
    constexpr int RPL = MODE == NVFP4 ? 4 : 2;  // rows per load
    if (rmin > 16 && (rmax == 20 || rmax == 24)) {
      if (rmax == 20) return launch_qf<MODE, M, 10, 1, 1, 1, false, 4 / RPL>(a, w2, s2, grid, F, st);
      return launch_qf<MODE, M, 10, 1, 1, 1, false, 8 / RPL>(a, w2, s2, grid, F, st);
    }
  }
  if constexpr (MODE == NVFP4 && !PARTS) {
    const int sl = qf_short_last(a, grid, NMAT == 2 ? 8 : 16);
    if constexpr (NMAT == 1) {
      if (sl == 1) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 1>(a, w2, s2, grid, F, st);
      if (sl == 2) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 2>(a, w2, s2, grid, F, st);
      if (sl == 3) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 3>(a, w2, s2, grid, F, st);
    } else {
      if (sl == 1) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 1>(a, w2, s2, grid, F, st);
    }
  }
  // mxfp8 (the model's shapes: 2, 4 or 5 of 8 loads; the MLP form measured no faster)
  if constexpr (MODE == MXFP8 && NMAT == 1 && !PARTS && M <= 8) {
    const int sl = qf_short_last(a, grid, 16, 3, 2);
    if (sl == 2) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 2>(a, w2, s2, grid, F, st);
    if (sl == 4) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 4>(a, w2, s2, grid, F, st);
    if (sl == 5) return launch_qf<MODE, M, 10, NMAT, 1, 1, false, 0, 5>(a, w2, s2, grid, F, st);
  }
  return launch_qf<MODE, M, 10, NMAT, 1, 1, PARTS>(a, w2, s2, grid, F, st);
}

template <int NMAT, bool PARTS = false>
static hipError_t launch_qf_any(const QmmArgs &a, const uint8_t *w2, const uint8_t *s2, hipStream_t st) {
  const int cus = qf_cus();
  if (cus == 0) return hipErrorNoDevice;
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int nrb = qf_nrb(a, cus, NMAT);
  const int F = qf_flush_rows(a, nrb);
  if (qf_shape(a.K).P > 1 && F < nrb) return hipErrorInvalidValue;
  if (a.mode == NVFP4) {
    if (a.M == 1) return launch_qf_d<NVFP4, 1, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
    return launch_qf_d<NVFP4, 2, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
  }
  if constexpr (NMAT == 1 && !PARTS) {  // (grouped calls and the MLP form run M <= 4)
    switch (a.M) {
      case 5: return launch_qf_d<MXFP8, 5, 1>(a, w2, s2, grid, F, nrb, st);
      case 6: return launch_qf_d<MXFP8, 6, 1>(a, w2, s2, grid, F, nrb, st);
      case 7: return launch_qf_d<MXFP8, 7, 1>(a, w2, s2, grid, F, nrb, st);
      case 8: return launch_qf_d<MXFP8, 8, 1>(a, w2, s2, grid, F, nrb, st);
      case 9: return launch_qf_d<MXFP8, 9, 1>(a, w2, s2, grid, F, nrb, st);
      case 10: return launch_qf_d<MXFP8, 10, 1>(a, w2, s2, grid, F, nrb, st);
      case 11: return launch_qf_d<MXFP8, 11, 1>(a, w2, s2, grid, F, nrb, st);
      case 12: return launch_qf_d<MXFP8, 12, 1>(a, w2, s2, grid, F, nrb, st);
      case 13: return launch_qf_d<MXFP8, 13, 1>(a, w2, s2, grid, F, nrb, st);
      case 14: return launch_qf_d<MXFP8, 14, 1>(a, w2, s2, grid, F, nrb, st);
      case 15: return launch_qf_d<MXFP8, 15, 1>(a, w2, s2, grid, F, nrb, st);
      case 16: return launch_qf_d<MXFP8, 16, 1>(a, w2, s2, grid, F, nrb, st);
      default: break;
    }
  }
  switch (a.M) {
    case 1: return launch_qf_d<MXFP8, 1, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
    case 2: return launch_qf_d<MXFP8, 2, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
    case 3: return launch_qf_d<MXFP8, 3, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
    default: return launch_qf_d<MXFP8, 4, NMAT, PARTS>(a, w2, s2, grid, F, nrb, st);
  }
}

// nvfp4 on the 32x32x64 form: 32-row blocks, one unit in flight per wave.
template <int M, int Q, int P, int NMAT, bool PARTS = false, int LU = 8, int SL = 0>
static hipError_t launch_q32(const QmmArgs &a, const uint8_t *w2, const uint8_t *s2, int grid, int F,
                             hipStream_t st) {
  auto kern = qmv_mfma32_kernel<M, Q, P, NMAT, PARTS, LU, SL>;
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t e = ensure_dynamic_lds(lds_set, (const void *)kern, 160 * 1024);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * Q), q32_lds_bytes(M, Q, F), st, a.N, a.K, F, a.N / grid,
                     a.N % grid, (const uint16_t *)a.x, a.w, a.s, w2, s2, yout_of(a));
  return hipGetLastError();
}

// Units per workgroup: row blocks of 32 rows (16 output rows in the MLP form).
static int q32_nrb(const QmmArgs &a, int cus, int nmat = 1) {
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int rb = nmat == 2 ? 16 : 32;
  return ((a.N + grid - 1) / grid + rb - 1) / rb;
}

static int q32_flush_rows(const QmmArgs &a, int nrb) {
  int F = nrb < Q32_FLUSH_MAX ? nrb : Q32_FLUSH_MAX;
  while (F > 1 && q32_lds_bytes(a.M, qf_shape(a.K).Q, F) > QF_LDS_MAX) --F;
  return F;
}

static bool q32_ok(const QmmArgs &a) {
  // (x of 5-8 rows at K = 5120 / 6144 runs the dequantizing kernel, faster than this form's
  // two A operands per chunk from N = 1024)
  if (a.mode != NVFP4 || a.x_f32 || a.M < 1 || a.M > 4 || a.N < 16) return false;
  const QfShape g = qf_shape(a.K);
  if (g.Q == 0 || qf_cus() == 0) return false;
  if (g.P > 1 && q32_flush_rows(a, q32_nrb(a, qf_cus())) < q32_nrb(a, qf_cus())) return false;
  if ((int64_t)a.N * (a.K / 2) >= ((int64_t)1 << 32)) return false;  // 32-bit offsets within W
  return ((((uintptr_t)a.x) | ((uintptr_t)a.w) | ((uintptr_t)a.s)) & 15) == 0;
}

// the plain 32-row form for K's (Q, P), with the loads a unit makes: at most 28 rows
// per workgroup (one row block; 5120 rows: 20) load only those rows
template <int M, int Q, int P>
static hipError_t launch_q32_lu(const QmmArgs &a, int grid, int F, hipStream_t st) {
  const int rows = a.N / grid + (a.N % grid ? 1 : 0), lu = (rows + 3) / 4;
  if constexpr (M >= 3) {
    if (lu <= 5) return launch_q32<M, Q, P, 1, false, 5>(a, a.w, a.s, grid, F, st);
    if (lu == 6) return launch_q32<M, Q, P, 1, false, 6>(a, a.w, a.s, grid, F, st);
    if (lu == 7) return launch_q32<M, Q, P, 1, false, 7>(a, a.w, a.s, grid, F, st);
  }
  if constexpr (P == 1 && M >= 3) {  // a short last row block of 2 or more
    switch (qf_short_last(a, grid, 32, 2)) {
      case 1: return launch_q32<M, Q, P, 1, false, 8, 1>(a, a.w, a.s, grid, F, st);
      case 2: return launch_q32<M, Q, P, 1, false, 8, 2>(a, a.w, a.s, grid, F, st);
      case 3: return launch_q32<M, Q, P, 1, false, 8, 3>(a, a.w, a.s, grid, F, st);
      case 4: return launch_q32<M, Q, P, 1, false, 8, 4>(a, a.w, a.s, grid, F, st);
      case 5: return launch_q32<M, Q, P, 1, false, 8, 5>(a, a.w, a.s, grid, F, st);
      case 6: return launch_q32<M, Q, P, 1, false, 8, 6>(a, a.w, a.s, grid, F, st);
      case 7: return launch_q32<M, Q, P, 1, false, 8, 7>(a, a.w, a.s, grid, F, st);
      default: break;
    }
  }
  return launch_q32<M, Q, P, 1>(a, a.w, a.s, grid, F, st);
}

template <int M>
static hipError_t launch_q32_k(const QmmArgs &a, QfShape g, int grid, int F, hipStream_t st) {
  if (g.P == 3) return launch_q32_lu<M, 12, 3>(a, grid, F, st);
  if (g.P == 2) return launch_q32_lu<M, 10, 2>(a, grid, F, st);
  if (g.Q == 12) return launch_q32_lu<M, 12, 1>(a, grid, F, st);
  return launch_q32_lu<M, 10, 1>(a, grid, F, st);
}

static hipError_t launch_q32_any(const QmmArgs &a, hipStream_t st) {
  if (!q32_ok(a)) return hipErrorInvalidValue;
  const int cus = qf_cus();
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int nrb = q32_nrb(a, cus);
  const int F = q32_flush_rows(a, nrb);
  const QfShape g = qf_shape(a.K);
  const uint8_t *w2 = a.w, *s2 = a.s;  // unused in the plain form
  if (a.parts) {  // grouped calls: K = 5120, M = 3-4
    if (g.Q != 10 || g.P != 1 || a.M < 3 || a.M > 4) return hipErrorInvalidValue;
    return a.M == 3 ? launch_q32<3, 10, 1, 1, true>(a, w2, s2, grid, F, st)
                    : launch_q32<4, 10, 1, 1, true>(a, w2, s2, grid, F, st);
  }
  switch (a.M) {
    case 1: return launch_q32_k<1>(a, g, grid, F, st);
    case 2: return launch_q32_k<2>(a, g, grid, F, st);
    case 3: return launch_q32_k<3>(a, g, grid, F, st);
    default: return launch_q32_k<4>(a, g, grid, F, st);
  }
}

// The MLP form at nvfp4 M = 3-4 (K = 5120, one pass).
static bool q32_mlp_ok(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up) {
  return a.M >= 3 && a.M <= 4 && q32_ok(a) && qf_shape(a.K).P == 1 && ((((uintptr_t)w_up) | ((uintptr_t)s_up)) & 15) == 0;
}

static hipError_t launch_q32_mlp(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st) {
  if (!q32_mlp_ok(a, w_up, s_up)) return hipErrorInvalidValue;
  const int cus = qf_cus();
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int nrb = q32_nrb(a, cus, 2);
  const int F = q32_flush_rows(a, nrb);
  switch (qf_short_last(a, grid, 16, 2)) {  // a short last row block of 2 or more
    case 1: return a.M == 3 ? launch_q32<3, 10, 1, 2, false, 8, 1>(a, w_up, s_up, grid, F, st)
                            : launch_q32<4, 10, 1, 2, false, 8, 1>(a, w_up, s_up, grid, F, st);
    case 2: return a.M == 3 ? launch_q32<3, 10, 1, 2, false, 8, 2>(a, w_up, s_up, grid, F, st)
                            : launch_q32<4, 10, 1, 2, false, 8, 2>(a, w_up, s_up, grid, F, st);
    case 3: return a.M == 3 ? launch_q32<3, 10, 1, 2, false, 8, 3>(a, w_up, s_up, grid, F, st)
                            : launch_q32<4, 10, 1, 2, false, 8, 3>(a, w_up, s_up, grid, F, st);
    default: break;
  }
  if (a.M == 3) return launch_q32<3, 10, 1, 2>(a, w_up, s_up, grid, F, st);
  return launch_q32<4, 10, 1, 2>(a, w_up, s_up, grid, F, st);
}

// Row blocks per partial-sum flush of the dequantizing kernel: as many as fit the LDS.
static int qd_flush_rows(int nrb, int Q) {
  int F = nrb < QD_FLUSH_MAX ? nrb : QD_FLUSH_MAX;
  while (F > 1 && qd_lds_bytes(Q, F) > QF_LDS_MAX) --F;
  return F;
}

template <int Q>
static hipError_t launch_qd(const QmmArgs &a, int grid, int F, hipStream_t st) {
  auto kern = qmv_deq16_kernel<Q>;
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t e = ensure_dynamic_lds(lds_set, (const void *)kern, 160 * 1024);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * Q), qd_lds_bytes(Q, F), st, a.N, a.K, a.M, F, a.N / grid,
                     a.N % grid, (const uint16_t *)a.x, a.w, a.s, (uint16_t *)a.y);
  return hipGetLastError();
}

static hipError_t launch_qd_any(const QmmArgs &a, hipStream_t st) {
  if (!qd_ok(a) || a.parts) return hipErrorInvalidValue;
  const int cus = qf_cus();
  const int rbs = (a.N + 15) / 16;
  const int grid = rbs < cus ? rbs : cus;
  const int Q = qf_shape(a.K).Q;
  const int F = qd_flush_rows(qf_nrb(a, cus), Q);
  return Q == 12 ? launch_qd<12>(a, grid, F, st) : launch_qd<10>(a, grid, F, st);
}

hipError_t launch_qmv_mfma(const QmmArgs &a, hipStream_t st) {
  if (!qmv_mfma_ok(a)) return hipErrorInvalidValue;
  if (a.mode == NVFP4 && a.M >= 5 && qd_ok(a)) return launch_qd_any(a, st);
  if (a.mode == NVFP4 && a.M > 2) return launch_q32_any(a, st);
  if (a.parts) return a.K == 5120 ? launch_qf_any<1, true>(a, a.w, a.s, st) : hipErrorInvalidValue;
  return launch_qf_any<1>(a, a.w, a.s, st);
}

// Grouped calls on these kernels: K = 5120 (not the dequantizing kernel).
bool qmv_mfma_parts_ok(const QmmArgs &a) { return qmv_mfma_ok(a) && a.K == 5120 && !(a.mode == NVFP4 && a.M > 4); }

hipError_t launch_qmv_mfma_mlp(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st) {
  if (!qmv_mfma_mlp_ok(a, w_up, s_up)) return hipErrorInvalidValue;
  if (a.mode == NVFP4 && a.M > 2) return launch_q32_mlp(a, w_up, s_up, st);
  return launch_qf_any<2>(a, w_up, s_up, st);
}

}  // namespace qmm
