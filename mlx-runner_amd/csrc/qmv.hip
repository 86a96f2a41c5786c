// Decode / speculative-verify quantized matmul (M = 1..8): y[m,n] = sum_k x[m,k] * deq(W)[n,k].
//
// The shapes this serves are mlx-runner's per-token qmm calls (src/model.zig:906-914,
// :929-979, :1066-1074, :1230, :1309; M = 1 decode, 2-3 MTP verify).  They are
// HBM-bound: every weight byte is read once.
//
// Mapping (gfx950, wave64):
//   * one wave owns a tile of R consecutive rows of W (contiguous in HBM);
//   * lane l walks the 16-byte chunks c = l, l+64, ... of each row, so every
//     load instruction reads 1 KiB of contiguous weights (global_load_dwordx4);
//   * the R rows share each x chunk (x read once per R rows, from L1/L2);
//   * elements are unpacked in registers with the gfx950 converters
//     (v_cvt_scalef32_pk_bf16_fp4 / _fp8, unit scale), multiplied with bf16
//     x pairs by v_dot2_f32_bf16 into a per-group fp32 partial, and the group
//     scale (E4M3 for nvfp4, E8M0 for mxfp8) is applied once per group;
//   * the R*M partials are reduced across the wave by xor-shuffles and lane
//     (r*M + m) stores y[m, n0 + r], rounded to bf16 (RNE) or kept f32.
// A 16-byte chunk holds 32 nvfp4 elements (2 groups) or 16 mxfp8 elements
// (half a group).
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

template <int MODE, int M, int R, bool XF32>
__global__ __launch_bounds__(64) void qmv_kernel(const void *__restrict__ xv, const uint8_t *__restrict__ w,
                                                 const uint8_t *__restrict__ s, void *__restrict__ yv, int N,
                                                 int K) {
  const int lane = threadIdx.x;
  const int n0 = blockIdx.x * R;
  const int64_t row_bytes = (MODE == MXFP8) ? (int64_t)K : (int64_t)(K >> 1);
  const int C = (int)(row_bytes >> 4);                   // 16-byte chunks per row
  const int spr = (MODE == MXFP8) ? (K >> 5) : (K >> 4); // scale bytes per row

  const uint8_t *wrow[R];
  const uint8_t *srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int n = n0 + r < N ? n0 + r : N - 1;  // clamp: tail rows load row N-1, results dropped
    wrow[r] = w + (int64_t)n * row_bytes;
    srow[r] = s + (int64_t)n * spr;
  }

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

  for (int c = lane; c < C; c += 64) {
    uint4 q[R];
    uint32_t sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      q[r] = load_stream16(wrow[r] + ((int64_t)c << 4));
      if (MODE == NVFP4)
        sc[r] = *(const uint16_t *)(srow[r] + 2 * c);
      else
        sc[r] = srow[r][c >> 1];
    }
    if constexpr (!XF32) {
      const uint16_t *x = (const uint16_t *)xv;
      constexpr int XW = (MODE == NVFP4) ? 16 : 8;  // x dwords per chunk
      uint32_t xw[M][XW];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4 *xp = (const uint4 *)(x + (int64_t)m * K + (int64_t)c * (MODE == NVFP4 ? 32 : 16));
#pragma unroll
        for (int j = 0; j < XW / 4; ++j) {
          uint4 t = xp[j];
          xw[m][4 * j + 0] = t.x;
          xw[m][4 * j + 1] = t.y;
          xw[m][4 * j + 2] = t.z;
          xw[m][4 * j + 3] = t.w;
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t d[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
        if constexpr (MODE == NVFP4) {
          bf16x2_t wb[16];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[4 * j + 0] = fp4x2_to_bf16x2<0>(d[j]);
            wb[4 * j + 1] = fp4x2_to_bf16x2<1>(d[j]);
            wb[4 * j + 2] = fp4x2_to_bf16x2<2>(d[j]);
            wb[4 * j + 3] = fp4x2_to_bf16x2<3>(d[j]);
          }
          float s0 = __builtin_amdgcn_cvt_f32_fp8((int)sc[r], 0);
          float s1 = __builtin_amdgcn_cvt_f32_fp8((int)sc[r], 1);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g0 = 0.f, g1 = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g0 = dot2_bf16(wb[j], xw[m][j], g0);
#pragma unroll
            for (int j = 8; j < 16; ++j) g1 = dot2_bf16(wb[j], xw[m][j], g1);
            acc[r][m] = __builtin_fmaf(g0, s0, acc[r][m]);
            acc[r][m] = __builtin_fmaf(g1, s1, acc[r][m]);
          }
        } else {
          bf16x2_t wb[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[2 * j + 0] = fp8x2_to_bf16x2<false>(d[j]);
            wb[2 * j + 1] = fp8x2_to_bf16x2<true>(d[j]);
          }
          float s0 = e8m0_to_f32(sc[r]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g = dot2_bf16(wb[j], xw[m][j], g);
            acc[r][m] = __builtin_fmaf(g, s0, acc[r][m]);
          }
        }
      }
    } else {
      const float *x = (const float *)xv;
      constexpr int EPC = (MODE == NVFP4) ? 32 : 16;  // elements per chunk
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t d[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
        float wf[EPC];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (MODE == NVFP4) {
            f32x2_t a = fp4x2_to_f32x2<0>(d[j]), b = fp4x2_to_f32x2<1>(d[j]);
            f32x2_t e = fp4x2_to_f32x2<2>(d[j]), f = fp4x2_to_f32x2<3>(d[j]);
            wf[8 * j + 0] = a.x; wf[8 * j + 1] = a.y; wf[8 * j + 2] = b.x; wf[8 * j + 3] = b.y;
            wf[8 * j + 4] = e.x; wf[8 * j + 5] = e.y; wf[8 * j + 6] = f.x; wf[8 * j + 7] = f.y;
          } else {
            f32x2_t a = fp8x2_to_f32x2<false>(d[j]), b = fp8x2_to_f32x2<true>(d[j]);
            wf[4 * j + 0] = a.x; wf[4 * j + 1] = a.y; wf[4 * j + 2] = b.x; wf[4 * j + 3] = b.y;
          }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float *xp = x + (int64_t)m * K + (int64_t)c * EPC;
          if constexpr (MODE == NVFP4) {
            float g0 = 0.f, g1 = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) g0 = __builtin_fmaf(xp[i], wf[i], g0);
#pragma unroll
            for (int i = 16; i < 32; ++i) g1 = __builtin_fmaf(xp[i], wf[i], g1);
            acc[r][m] = __builtin_fmaf(g0, __builtin_amdgcn_cvt_f32_fp8((int)sc[r], 0), acc[r][m]);
            acc[r][m] = __builtin_fmaf(g1, __builtin_amdgcn_cvt_f32_fp8((int)sc[r], 1), acc[r][m]);
          } else {
            float g = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) g = __builtin_fmaf(xp[i], wf[i], g);
            acc[r][m] = __builtin_fmaf(g, e8m0_to_f32(sc[r]), acc[r][m]);
          }
        }
      }
    }
  }

  float out = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = wave_sum(acc[r][m]);
      out = (lane == r * M + m) ? t : out;
    }
  if (lane < R * M) {
    int r = lane / M, m = lane % M;
    if (n0 + r < N) {
      if constexpr (XF32)
        ((float *)yv)[(int64_t)m * N + n0 + r] = out;
      else
        ((uint16_t *)yv)[(int64_t)m * N + n0 + r] = f32_to_bf16_rne(out);
    }
  }
}

// Any-shape fallback (K a multiple of the group, row bytes not a multiple of 16):
// one wave per (row, m), lanes stride elements; exact integer decoders.  Each term
// is (x * elem) * scale in one fused step, so a weight whose f32 dequant would
// overflow still multiplies x as its true value (0 * it is 0), as in the other
// kernels, which scale each group's partial sum.
template <int MODE, bool XF32>
__global__ __launch_bounds__(64) void qmv_generic_kernel(const void *__restrict__ xv, const uint8_t *__restrict__ w,
                                                         const uint8_t *__restrict__ s, void *__restrict__ yv,
                                                         int M, int N, int K) {
  const int lane = threadIdx.x;
  const int n = blockIdx.x, m = blockIdx.y;
  const int g = (MODE == MXFP8) ? 32 : 16;
  const uint32_t *wr = (const uint32_t *)(w + (int64_t)n * (MODE == MXFP8 ? K : K / 2));
  const uint8_t *sr = s + (int64_t)n * (K / g);
  float acc = 0.f;
  for (int k = lane; k < K; k += 64) {
    float e, sc;
    if (MODE == MXFP8) {
      e = e4m3_to_f32_int((wr[k >> 2] >> (8 * (k & 3))) & 0xFFu);
      sc = e8m0_to_f32(sr[k >> 5]);
    } else {
      e = e2m1_to_f32_int((wr[k >> 3] >> (4 * (k & 7))) & 0xFu);
      sc = e4m3_to_f32_int(sr[k >> 4]);
    }
    float xk = XF32 ? ((const float *)xv)[(int64_t)m * K + k] : bf16_to_f32(((const uint16_t *)xv)[(int64_t)m * K + k]);
    acc = __builtin_fmaf(xk * e, sc, acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if (XF32)
      ((float *)yv)[(int64_t)m * N + n] = acc;
    else
      ((uint16_t *)yv)[(int64_t)m * N + n] = f32_to_bf16_rne(acc);
  }
}

// ---------------------------------------------------------------- bf16 decode kernel
//
// 512-thread blocks; wave w of block b owns rows n0 = (8b + w) * R ... + R.  K is
// walked in segments of ISEG chunk iterations: every lane issues all R x ISEG
// 16-byte weight loads (plus their scale bytes) of a segment at once, with the
// next segment's loads in flight while the current one is computed.  x is staged
// once per block in LDS, each chunk's x padded (64 -> 80 bytes for nvfp4, 32 -> 48
// for mxfp8) so the 16-byte reads of consecutive lanes land in distinct banks; its
// global loads are issued before the weight loads so that staging waits only for
// them.  When M * K is too large for LDS, x is read from global (L1/L2).
constexpr int QMV_WAVES = 8;

template <int MODE>
struct XLayout {
  static constexpr int EPC = MODE == NVFP4 ? 32 : 16;     // elements per 16-byte weight chunk
  static constexpr int XBYTES = EPC * 2;                  // bf16 x bytes per chunk
  static constexpr int PITCH = MODE == NVFP4 ? 80 : 48;   // padded LDS bytes per chunk
  static constexpr int PIECES = XBYTES / 16;              // uint4 pieces per chunk
};

inline size_t qmv_lds_bytes(int mode, int M, int K) {
  const int C = mode == MXFP8 ? K / 16 : K / 32;
  return (size_t)M * C * (mode == NVFP4 ? 80 : 48);
}
constexpr size_t QMV_LDS_MAX = 64 * 1024;

// MLP: the wave's two rows are row n of W (gate) and row n of W2 (up), and the
// output is silu(gate) * up with the reference's bf16 roundings (silu_mul_bf16).
// WV: waves per workgroup (QMV_WAVES, or 5 where that spreads the rows evenly over the CUs).
template <int MODE, int M, int R, int ISEG, int XP, bool DB, bool MLP = false, bool PARTS = false, int WV = QMV_WAVES>
__global__ __launch_bounds__(64 * WV) void qmv_bf16_kernel(int N, int K, const uint16_t *__restrict__ x,
                                                                  const uint8_t *__restrict__ w,
                                                                  const uint8_t *__restrict__ s,
                                                                  const uint8_t *__restrict__ w2,
                                                                  const uint8_t *__restrict__ s2, const YOut yo) {
  using L = XLayout<MODE>;
  constexpr int THREADS = 64 * WV;
  constexpr bool XLDS = XP > 0;  // XP: x pieces staged per thread (2 or 4; 0: x read from global)
  static_assert(XP == 0 || XP == 2 || XP == 4, "x staging supports 2 or 4 pieces per thread");
  static_assert(!MLP || R == 2, "the MLP form pairs one gate row with one up row");
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * WV + wave) * (MLP ? 1 : R);
  const int64_t row_bytes = (MODE == MXFP8) ? (int64_t)K : (int64_t)(K >> 1);
  const int C = (int)(row_bytes >> 4);
  const int spr = (MODE == MXFP8) ? (K >> 5) : (K >> 4);
  const uint8_t *wrow[R];
  const uint8_t *srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (MLP) {
      const int n = n0 < N ? n0 : N - 1;
      wrow[r] = (r == 0 ? w : w2) + (int64_t)n * row_bytes;
      srow[r] = (r == 0 ? s : s2) + (int64_t)n * spr;
    } else {
      const int n = n0 + r < N ? n0 + r : N - 1;  // tail rows re-read row N-1; results dropped
      wrow[r] = w + (int64_t)n * row_bytes;
      srow[r] = s + (int64_t)n * spr;
    }
  }

  // 1) x staging loads first: the LDS write below then waits only for these,
  //    not for the weight loads issued after them.
  const int pieces = M * C * L::PIECES;  // host guarantees pieces <= XP * THREADS
  // x pieces are contiguous in global memory: piece p is (m, c, j) with p = (m * C + c) * PIECES + j
  auto xload = [&](int k) __attribute__((always_inline)) {
    const int p = threadIdx.x + THREADS * k;
    return ((const uint4 *)x)[p < pieces ? p : pieces - 1];
  };
  uint4 xr0, xr1, xr2, xr3;
  if constexpr (XLDS) {
    xr0 = xload(0);
    xr1 = xload(1);
    if constexpr (XP > 2) {
      xr2 = xload(2);
      xr3 = xload(3);
    }
  }
  // keep every x load ahead of the weight loads (the wait counter counts in issue order: an
  // x load scheduled after them would make the LDS store below wait for all of them)
  __builtin_amdgcn_sched_barrier(0);

  // 2) weight loads of a segment: clamped addresses, no per-load branches
  auto load_seg = [&](int seg, uint4 (&q)[ISEG][R], uint32_t (&sc)[ISEG][R]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < ISEG; ++i) {
      int c = seg * 64 * ISEG + lane + 64 * i;
      c = c < C ? c : C - 1;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        q[i][r] = load_stream16(wrow[r] + ((int64_t)c << 4));
        sc[i][r] = (MODE == NVFP4) ? (uint32_t) * (const uint16_t *)(srow[r] + 2 * c) : (uint32_t)srow[r][c >> 1];
      }
    }
  };

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

  auto compute_seg = [&](int seg, const uint4 (&q)[ISEG][R], const uint32_t (&sc)[ISEG][R]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < ISEG; ++i) {
      const int craw = seg * 64 * ISEG + lane + 64 * i;
      const bool valid = craw < C;
      const int c = valid ? craw : C - 1;
      constexpr int XW = L::XBYTES / 4;
      uint32_t xw[M][XW];
#pragma unroll
      for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < L::PIECES; ++j) {
          const uint4 t = XLDS ? *(const uint4 *)(xs + (m * C + c) * L::PITCH + 16 * j)
                               : ((const uint4 *)(x + (int64_t)m * K + (int64_t)c * L::EPC))[j];
          xw[m][4 * j + 0] = t.x;
          xw[m][4 * j + 1] = t.y;
          xw[m][4 * j + 2] = t.z;
          xw[m][4 * j + 3] = t.w;
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t d[4] = {q[i][r].x, q[i][r].y, q[i][r].z, q[i][r].w};
        if constexpr (MODE == NVFP4) {
          bf16x2_t wb[16];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[4 * j + 0] = fp4x2_to_bf16x2<0>(d[j]);
            wb[4 * j + 1] = fp4x2_to_bf16x2<1>(d[j]);
            wb[4 * j + 2] = fp4x2_to_bf16x2<2>(d[j]);
            wb[4 * j + 3] = fp4x2_to_bf16x2<3>(d[j]);
          }
          const float s0 = __builtin_amdgcn_cvt_f32_fp8((int)sc[i][r], 0);
          const float s1 = __builtin_amdgcn_cvt_f32_fp8((int)sc[i][r], 1);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g0 = 0.f, g1 = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g0 = dot2_bf16(wb[j], xw[m][j], g0);
#pragma unroll
            for (int j = 8; j < 16; ++j) g1 = dot2_bf16(wb[j], xw[m][j], g1);
            const float t = __builtin_fmaf(g1, s1, g0 * s0);
            acc[r][m] += valid ? t : 0.f;
          }
        } else {
          bf16x2_t wb[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[2 * j + 0] = fp8x2_to_bf16x2<false>(d[j]);
            wb[2 * j + 1] = fp8x2_to_bf16x2<true>(d[j]);
          }
          const float s0 = e8m0_to_f32(sc[i][r]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g = dot2_bf16(wb[j], xw[m][j], g);
            acc[r][m] += valid ? g * s0 : 0.f;
          }
        }
      }
    }
  };

  const int nseg = (C + 64 * ISEG - 1) / (64 * ISEG);
  uint4 qa[ISEG][R], qb[DB ? ISEG : 1][R];
  uint32_t sa[ISEG][R], sb[DB ? ISEG : 1][R];
  load_seg(0, qa, sa);
  if constexpr (DB) {
    if (nseg > 1) load_seg(1, qb, sb);
  }
  __builtin_amdgcn_sched_barrier(0);  // the weight loads stay ahead of the x staging barrier
  if constexpr (XLDS) {
    // piece (m, c, j) lands at (m * C + c) * PITCH + 16 j
    // unconditional: a thread past the last piece loaded that piece (the clamp in xload)
    // and stores the same bytes to its slot; no branch, so the compiler cannot sink the x
    // load into one behind the weight loads
    auto xstore = [&](int k, const uint4 &v) __attribute__((always_inline)) {
      int p = threadIdx.x + THREADS * k;
      p = p < pieces ? p : pieces - 1;
      const int mc = p / L::PIECES, j = p - mc * L::PIECES;
      *(uint4 *)(xs + mc * L::PITCH + 16 * j) = v;
    };
    xstore(0, xr0);
    xstore(1, xr1);
    if constexpr (XP > 2) {
      xstore(2, xr2);
      xstore(3, xr3);
    }
    // a barrier for the LDS stores only: __syncthreads() would also wait for every weight
    // load in flight (vmcnt(0)), so no chunk could be decoded before the last one landed.
    // The weight and scale pointers are operands of the asm, so the compiler keeps those
    // loads ahead of it (it would otherwise sink them past it, to their first use).
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::"s"(w), "s"(w2), "s"(s), "s"(s2) : "memory");
  }
  if constexpr (DB) {
    // two segments in flight: compute one while the next one's loads land
    for (int seg = 0; seg < nseg; seg += 2) {
      compute_seg(seg, qa, sa);
      if (seg + 2 < nseg) load_seg(seg + 2, qa, sa);
      if (seg + 1 < nseg) {
        compute_seg(seg + 1, qb, sb);
        if (seg + 3 < nseg) load_seg(seg + 3, qb, sb);
      }
    }
  } else {
    for (int seg = 0; seg < nseg; ++seg) {
      if (seg > 0) load_seg(seg, qa, sa);
      compute_seg(seg, qa, sa);
    }
  }

  if constexpr (MLP) {
    float out = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float g = wave_sum(acc[0][m]), u = wave_sum(acc[1][m]);
      out = (lane == m) ? silu_mul_bf16(g, u) : out;
    }
    if (lane < M && n0 < N) yo.y0[(int64_t)lane * N + n0] = f32_to_bf16_rne(out);
    return;
  }
  float out = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float t = wave_sum(acc[r][m]);
      out = (lane == r * M + m) ? t : out;
    }
  if (lane < R * M) {
    const int r = lane / M, m = lane % M;
    if (n0 + r < N) {
      const uint16_t v = f32_to_bf16_rne(out);
      if constexpr (PARTS)
        *yo.at(m, n0 + r) = v;
      else
        yo.y0[(int64_t)m * N + n0 + r] = v;
    }
  }
}

template <int MODE, int M, int R, int ISEG, bool DB, bool PARTS = false, int WV = QMV_WAVES>
static hipError_t launch_qmv_bf16_t(const QmmArgs &a, hipStream_t st) {
  const size_t lds = qmv_lds_bytes(MODE, M, a.K);
  const int C = MODE == MXFP8 ? a.K / 16 : a.K / 32;
  const int pieces = M * C * (MODE == NVFP4 ? 4 : 2);
  constexpr int T = 64 * WV;
  dim3 grid((a.N + R * WV - 1) / (R * WV));
  const uint16_t *x = (const uint16_t *)a.x;
  const YOut y = yout_of(a);
  if (lds <= QMV_LDS_MAX && pieces <= 2 * T)
    hipLaunchKernelGGL((qmv_bf16_kernel<MODE, M, R, ISEG, 2, DB, false, PARTS, WV>), grid, dim3(T), lds, st, a.N, a.K,
                       x, a.w, a.s, nullptr, nullptr, y);
  else if (lds <= QMV_LDS_MAX && pieces <= 4 * T)
    hipLaunchKernelGGL((qmv_bf16_kernel<MODE, M, R, ISEG, 4, DB, false, PARTS, WV>), grid, dim3(T), lds, st, a.N, a.K,
                       x, a.w, a.s, nullptr, nullptr, y);
  else
    hipLaunchKernelGGL((qmv_bf16_kernel<MODE, M, R, ISEG, 0, DB, false, PARTS, WV>), grid, dim3(T), 0, st, a.N, a.K, x,
                       a.w, a.s, nullptr, nullptr, y);
  return hipGetLastError();
}

// Whether 5-wave workgroups spread N rows (one per wave) over the CUs more evenly
// than 8-wave ones.  A CU takes whole workgroups, and the time is set by the CUs
// with the most rows: N = 5120 in 640 8-wave workgroups leaves half the CUs three
// (24 rows) and half two, in 1024 5-wave ones every CU gets four (20 rows).
// Measured at mxfp8 N = K = 5120 (one box, per-wave timestamps): 6.91 -> 6.57 us;
// 10-wave workgroups (two per CU) gained nothing and 4-wave ones slightly less.
static bool qmv_five_waves(int N) {
  const int cus = device_cu_count();
  if (cus <= 0) return false;
  auto max_rows = [&](int wv) {  // rows of the most loaded CU
    const int64_t grid = (N + (int64_t)wv - 1) / wv;
    return (grid + cus - 1) / cus * (int64_t)wv;
  };
  return max_rows(5) < max_rows(QMV_WAVES);
}

// Rows per wave: two where the grid stays large (the gate+up shape, N = 34816:
// 18.3 us against 19.6 us at one row; the lm_head), one for short N, where two
// rows leave too few blocks (N = 5120 at M = 1: 8.4 us against 6.8 us).
// Single-segment shapes only (C <= 320 chunks: nvfp4 K <= 10240, mxfp8 K <= 5120);
// longer rows use the long-row kernel.
template <int MODE, int M, bool PARTS>
static hipError_t launch_qmv_bf16_p(const QmmArgs &a, hipStream_t st) {
  const int C = MODE == MXFP8 ? a.K / 16 : a.K / 32;
  if (M == 1 && a.N < 16384) {
    if (qmv_five_waves(a.N)) {
      if (C <= 3 * 64) return launch_qmv_bf16_t<MODE, M, 1, 3, false, PARTS, 5>(a, st);
      return launch_qmv_bf16_t<MODE, M, 1, 5, false, PARTS, 5>(a, st);
    }
    if (C <= 3 * 64) return launch_qmv_bf16_t<MODE, M, 1, 3, false, PARTS>(a, st);
    return launch_qmv_bf16_t<MODE, M, 1, 5, false, PARTS>(a, st);
  }
  if (C <= 3 * 64) return launch_qmv_bf16_t<MODE, M, 2, 3, false, PARTS>(a, st);
  return launch_qmv_bf16_t<MODE, M, 2, 5, false, PARTS>(a, st);
}

// (the grouped instances, with the output part lookup, only for grouped calls)
template <int MODE, int M>
static hipError_t launch_qmv_bf16_m(const QmmArgs &a, hipStream_t st) {
  return a.parts ? launch_qmv_bf16_p<MODE, M, true>(a, st) : launch_qmv_bf16_p<MODE, M, false>(a, st);
}

template <int MODE>
static hipError_t launch_qmv_bf16(const QmmArgs &a, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_qmv_bf16_m<MODE, 1>(a, st);
    case 2: return launch_qmv_bf16_m<MODE, 2>(a, st);
    case 3: return launch_qmv_bf16_m<MODE, 3>(a, st);
    case 4: return launch_qmv_bf16_m<MODE, 4>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int MODE, int M>
static hipError_t launch_qmv_mlp_m(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st) {
  const int C = MODE == MXFP8 ? a.K / 16 : a.K / 32;
  const size_t lds = qmv_lds_bytes(MODE, M, a.K);
  const int pieces = M * C * (MODE == NVFP4 ? 4 : 2);
  constexpr int T = 64 * QMV_WAVES;
  dim3 grid((a.N + QMV_WAVES - 1) / QMV_WAVES);
  const uint16_t *x = (const uint16_t *)a.x;
  const YOut y = yout_of(a);
#define QMV_MLP_LAUNCH(IS, XP)                                                                                 \
  hipLaunchKernelGGL((qmv_bf16_kernel<MODE, M, 2, IS, XP, false, true>), grid, dim3(T), XP ? lds : 0, st, a.N, a.K, \
                     x, a.w, a.s, w_up, s_up, y)
  if (C <= 3 * 64) {
    if (lds <= QMV_LDS_MAX && pieces <= 2 * T) QMV_MLP_LAUNCH(3, 2);
    else if (lds <= QMV_LDS_MAX && pieces <= 4 * T) QMV_MLP_LAUNCH(3, 4);
    else QMV_MLP_LAUNCH(3, 0);
  } else {
    if (lds <= QMV_LDS_MAX && pieces <= 2 * T) QMV_MLP_LAUNCH(5, 2);
    else if (lds <= QMV_LDS_MAX && pieces <= 4 * T) QMV_MLP_LAUNCH(5, 4);
    else QMV_MLP_LAUNCH(5, 0);
  }
#undef QMV_MLP_LAUNCH
  return hipGetLastError();
}

static bool qmv_single_segment(const QmmArgs &a) {
  const int C = a.mode == MXFP8 ? a.K / 16 : a.K / 32;
  return a.M <= 4 && C <= 5 * 64;
}

// ---------------------------------------------------------------- long-K decode kernel
//
// Rows too long for x to sit in registers (the down projection: K = 17408, only
// N = 5120 rows).  Read from L2 per chunk, x would cost four times the weight
// bytes, so each 512-thread block copies x once into LDS with LDS DMA
// (global_load_lds_dwordx4, issued after the first weight loads so the two
// latencies overlap).  The grid is a few 4-wave blocks per CU; each wave streams
// rows gw, gw + nw, ... (nw waves in the grid) in units of ISEG chunks per lane
// (a whole 544-chunk row is one unit at ISEG = 9), always with the next unit's
// loads in flight while the current one is computed, so the unpack math
// overlaps the memory stream instead of following it.  x sits in LDS unpadded: the
// 16-byte pieces of chunk c (4 for nvfp4, 2 for mxfp8) are stored permuted,
// piece j at slot j ^ xswz(c), so the reads of consecutive lanes (consecutive
// chunks, one piece each) fall in distinct banks.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void qmv_dma16(const void *g, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(l), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int MODE>
__device__ __forceinline__ int xswz(int c) {
  return MODE == NVFP4 ? ((c >> 1) ^ (c >> 2)) & 3 : ((c >> 2) ^ (c >> 3)) & 1;
}

constexpr int QLONG_WAVES = 4;

template <int MODE, int M, int ISEG, int R>
__global__ __launch_bounds__(64 * QLONG_WAVES) void qmv_long_kernel(int N, int K, const uint16_t *__restrict__ x,
                                                                    const uint8_t *__restrict__ w,
                                                                    const uint8_t *__restrict__ s, const YOut yo) {
  using L = XLayout<MODE>;
  constexpr int T = 64 * QLONG_WAVES;
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  const uint32_t xs0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)xs;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row_bytes = (MODE == MXFP8) ? (int64_t)K : (int64_t)(K >> 1);
  const int C = (int)(row_bytes >> 4);
  const int spr = (MODE == MXFP8) ? (K >> 5) : (K >> 4);
  // this wave's row groups (R rows each): gw, gw + nw, ...; the rows of group k are
  // R (gw + k nw) + [0, R); work unit u = (group u / nseg, segment u % nseg)
  const int gw = blockIdx.x * QLONG_WAVES + wave, nw = gridDim.x * QLONG_WAVES;
  const int nseg = (C + 64 * ISEG - 1) / (64 * ISEG);
  const int ngroups = (N + R - 1) / R;
  const int nrows = gw < ngroups ? (ngroups - 1 - gw) / nw + 1 : 0;
  const int units = nrows * nseg;

  auto load_unit = [&](int u, uint4 (&q)[ISEG][R], uint32_t (&sc)[ISEG][R]) __attribute__((always_inline)) {
    const int k = u / nseg, seg = u - k * nseg;
    const int64_t n0 = (int64_t)R * (gw + (int64_t)k * nw);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r < N ? n0 + r : N - 1;  // tail rows re-read row N - 1; results dropped
      const uint8_t *wr = w + n * row_bytes;
      const uint8_t *sr = s + n * spr;
#pragma unroll
      for (int i = 0; i < ISEG; ++i) {
        int c = seg * 64 * ISEG + lane + 64 * i;
        c = c < C ? c : C - 1;
        q[i][r] = load_stream16(wr + ((int64_t)c << 4));
        sc[i][r] = (MODE == NVFP4) ? (uint32_t) * (const uint16_t *)(sr + 2 * c) : (uint32_t)sr[c >> 1];
      }
    }
  };
  uint4 qa[ISEG][R], qb[ISEG][R];
  uint32_t sa[ISEG][R], sb[ISEG][R];
  if (units > 0) load_unit(0, qa, sa);
  if (units > 1) load_unit(1, qb, sb);

  // x -> LDS: slot p (16 bytes) of the M x C x PIECES slots <- piece (p & ~mask) | ((p & mask) ^ xswz(chunk))
  {
    constexpr int PM = L::PIECES - 1;
    const int slots = M * C * L::PIECES;
    for (int base = wave * 64; base < slots; base += T) {
      const int p = base + lane;
      const int mc = p / L::PIECES, c = mc % C, j = p & PM;
      const int src = (mc * L::PIECES) | (j ^ xswz<MODE>(c));
      if (p < slots) qmv_dma16(x + (int64_t)src * 8, xs0 + (uint32_t)base * 16);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

  auto compute_unit = [&](int u, const uint4 (&q)[ISEG][R], const uint32_t (&sc)[ISEG][R]) __attribute__((always_inline)) {
    const int k = u / nseg, seg = u - k * nseg;
#pragma unroll
    for (int i = 0; i < ISEG; ++i) {
      const int craw = seg * 64 * ISEG + lane + 64 * i;
      const bool valid = craw < C;
      const int c = valid ? craw : C - 1;
      constexpr int XW = L::XBYTES / 4;
      const int sw = xswz<MODE>(c);
      uint32_t xw[M][XW];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int j = 0; j < L::PIECES; ++j) {
          const uint4 v = *(const uint4 *)(xs + ((m * C + c) * L::PIECES + (j ^ sw)) * 16);
          xw[m][4 * j + 0] = v.x;
          xw[m][4 * j + 1] = v.y;
          xw[m][4 * j + 2] = v.z;
          xw[m][4 * j + 3] = v.w;
        }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t d[4] = {q[i][r].x, q[i][r].y, q[i][r].z, q[i][r].w};
        if constexpr (MODE == NVFP4) {
          bf16x2_t wb[16];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[4 * j + 0] = fp4x2_to_bf16x2<0>(d[j]);
            wb[4 * j + 1] = fp4x2_to_bf16x2<1>(d[j]);
            wb[4 * j + 2] = fp4x2_to_bf16x2<2>(d[j]);
            wb[4 * j + 3] = fp4x2_to_bf16x2<3>(d[j]);
          }
          const float s0 = __builtin_amdgcn_cvt_f32_fp8((int)sc[i][r], 0);
          const float s1 = __builtin_amdgcn_cvt_f32_fp8((int)sc[i][r], 1);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g0 = 0.f, g1 = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g0 = dot2_bf16(wb[j], xw[m][j], g0);
#pragma unroll
            for (int j = 8; j < 16; ++j) g1 = dot2_bf16(wb[j], xw[m][j], g1);
            const float v = __builtin_fmaf(g1, s1, g0 * s0);
            acc[r][m] += valid ? v : 0.f;
          }
        } else {
          bf16x2_t wb[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wb[2 * j + 0] = fp8x2_to_bf16x2<false>(d[j]);
            wb[2 * j + 1] = fp8x2_to_bf16x2<true>(d[j]);
          }
          const float s0 = e8m0_to_f32(sc[i][r]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float g = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) g = dot2_bf16(wb[j], xw[m][j], g);
            acc[r][m] += valid ? g * s0 : 0.f;
          }
        }
      }
    }
    if (seg == nseg - 1) {  // rows done: reduce, lane r * M + m writes y[m, n0 + r], restart
      const int64_t n0 = (int64_t)R * (gw + (int64_t)k * nw);
      float out = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float v = wave_sum(acc[r][m]);
          out = lane == r * M + m ? v : out;
          acc[r][m] = 0.f;
        }
      if (lane < R * M && n0 + lane / M < N) yo.y0[(int64_t)(lane % M) * N + n0 + lane / M] = f32_to_bf16_rne(out);
    }
  };
  // two units in flight: compute one while the next one's loads land
  for (int u = 0; u < units; u += 2) {
    compute_unit(u, qa, sa);
    if (u + 2 < units) load_unit(u + 2, qa, sa);
    if (u + 1 < units) {
      compute_unit(u + 1, qb, sb);
      if (u + 3 < units) load_unit(u + 3, qb, sb);
    }
  }
}

inline size_t qmv_long_lds(int mode, int M, int K) { return (size_t)M * K * 2; }  // x, bf16, unpadded
// dynamic LDS cap: 160 KiB per CU minus room for the kernel's static reduction array
constexpr size_t QMV_LONG_LDS_MAX = 156 * 1024;

// Blocks per CU: as many as the CU's LDS holds copies of x (1 from M * K * 2 > 78 KiB).
template <int MODE, int M, int ISEG, int R, int PER_CU>
static hipError_t launch_qmv_long_t(const QmmArgs &a, hipStream_t st) {
  const size_t lds = qmv_long_lds(MODE, M, a.K);
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t e =
      ensure_dynamic_lds(lds_set, (const void *)qmv_long_kernel<MODE, M, ISEG, R>, (int)QMV_LONG_LDS_MAX);
  if (e != hipSuccess) return e;
  const int cus = device_cu_count();
  if (cus <= 0) return hipErrorNoDevice;
  const int per_cu = (int)(QMV_LONG_LDS_MAX / lds) < PER_CU ? (int)(QMV_LONG_LDS_MAX / lds) : PER_CU;
  const int want = ((a.N + R - 1) / R + QLONG_WAVES - 1) / QLONG_WAVES, have = cus * (per_cu > 0 ? per_cu : 1);
  dim3 grid(want < have ? want : have);
  hipLaunchKernelGGL((qmv_long_kernel<MODE, M, ISEG, R>), grid, dim3(64 * QLONG_WAVES), lds, st, a.N, a.K,
                     (const uint16_t *)a.x, a.w, a.s, yout_of(a));
  return hipGetLastError();
}

// ISEG and blocks per CU measured on the down projection (nvfp4, N = 5120, K = 17408):
// 12.1 / 16.2 / 22.5 us at M = 1 / 2 / 3.
template <int MODE>
static hipError_t launch_qmv_long(const QmmArgs &a, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_qmv_long_t<MODE, 1, 3, 1, 4>(a, st);
    case 2: return launch_qmv_long_t<MODE, 2, 5, 1, 2>(a, st);
    case 3: return launch_qmv_long_t<MODE, 3, 9, 1, 1>(a, st);
    case 4: return launch_qmv_long_t<MODE, 4, 9, 1, 1>(a, st);
    default: return hipErrorInvalidValue;
  }
}

static bool qmv_long_ok(const QmmArgs &a) {
  return !a.x_f32 && a.M <= 4 && qmv_long_lds(a.mode, a.M, a.K) <= QMV_LONG_LDS_MAX && (uintptr_t)a.x % 16 == 0;
}

template <int MODE, int M, int R, bool XF32>
static hipError_t launch_qmv_t(const QmmArgs &a, hipStream_t st) {
  dim3 grid((a.N + R - 1) / R);
  hipLaunchKernelGGL((qmv_kernel<MODE, M, R, XF32>), grid, dim3(64), 0, st, a.x, a.w, a.s, a.y, a.N, a.K);
  return hipGetLastError();
}

template <int MODE, bool XF32>
static hipError_t launch_qmv_mode(const QmmArgs &a, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_qmv_t<MODE, 1, 4, XF32>(a, st);
    case 2: return launch_qmv_t<MODE, 2, 4, XF32>(a, st);
    case 3: return launch_qmv_t<MODE, 3, 4, XF32>(a, st);
    case 4: return launch_qmv_t<MODE, 4, 4, XF32>(a, st);
    case 5: return launch_qmv_t<MODE, 5, 2, XF32>(a, st);
    case 6: return launch_qmv_t<MODE, 6, 2, XF32>(a, st);
    case 7: return launch_qmv_t<MODE, 7, 2, XF32>(a, st);
    case 8: return launch_qmv_t<MODE, 8, 2, XF32>(a, st);
    default: return hipErrorInvalidValue;
  }
}

bool qmv_fast_ok(const QmmArgs &a) {
  int64_t row_bytes = a.mode == MXFP8 ? a.K : a.K / 2;
  return a.M >= 1 && a.M <= QMV_MAX_M && row_bytes % 16 == 0 && a.K > 0 && a.N > 0;
}

hipError_t launch_qmv(const QmmArgs &a, hipStream_t st) {
  if (!qmv_fast_ok(a)) return hipErrorInvalidValue;
  if (!a.x_f32 && qmv_single_segment(a))
    return a.mode == MXFP8 ? launch_qmv_bf16<MXFP8>(a, st) : launch_qmv_bf16<NVFP4>(a, st);
  if (qmv_long_ok(a)) return a.mode == MXFP8 ? launch_qmv_long<MXFP8>(a, st) : launch_qmv_long<NVFP4>(a, st);
  if (a.mode == MXFP8) return a.x_f32 ? launch_qmv_mode<MXFP8, true>(a, st) : launch_qmv_mode<MXFP8, false>(a, st);
  return a.x_f32 ? launch_qmv_mode<NVFP4, true>(a, st) : launch_qmv_mode<NVFP4, false>(a, st);
}

// The kernels with grouped instances: the two MFMA forms at one pass and the
// bf16 GEMV, i.e. what run_qmm picks for bf16 x, M <= 4, 16-byte aligned x and
// W, at K = 5120 (MFMA) or single-segment rows (bf16 GEMV).
bool qmv_parts_ok(const QmmArgs &a) {
  if (a.x_f32 || a.M < 1 || a.M > 4 || a.N < 1 || a.K < 1) return false;
  if ((((uintptr_t)a.x) | ((uintptr_t)a.w)) & 15) return false;
  if (qmv_mfma_ok(a)) return qmv_mfma_parts_ok(a);
  return qmv_fast_ok(a) && qmv_single_segment(a);
}

bool qmv_mlp_ok(const QmmArgs &a) {
  return !a.x_f32 && a.M >= 1 && a.M <= 4 && qmv_fast_ok(a) && qmv_single_segment(a) &&
         (((uintptr_t)a.x | (uintptr_t)a.w) & 15) == 0;
}

hipError_t launch_qmv_mlp(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st) {
  if (!qmv_mlp_ok(a) || ((uintptr_t)w_up & 15) != 0) return hipErrorInvalidValue;
  const bool mx = a.mode == MXFP8;
  switch (a.M) {
    case 1: return mx ? launch_qmv_mlp_m<MXFP8, 1>(a, w_up, s_up, st) : launch_qmv_mlp_m<NVFP4, 1>(a, w_up, s_up, st);
    case 2: return mx ? launch_qmv_mlp_m<MXFP8, 2>(a, w_up, s_up, st) : launch_qmv_mlp_m<NVFP4, 2>(a, w_up, s_up, st);
    case 3: return mx ? launch_qmv_mlp_m<MXFP8, 3>(a, w_up, s_up, st) : launch_qmv_mlp_m<NVFP4, 3>(a, w_up, s_up, st);
    default: return mx ? launch_qmv_mlp_m<MXFP8, 4>(a, w_up, s_up, st) : launch_qmv_mlp_m<NVFP4, 4>(a, w_up, s_up, st);
  }
}

// ---------------------------------------------------------------- silu(g) * u, element-wise

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T *__restrict__ g, const T *__restrict__ u,
                                                       T *__restrict__ h, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if constexpr (sizeof(T) == 2) {
      h[i] = f32_to_bf16_rne(silu_mul_bf16(bf16_to_f32(g[i]), bf16_to_f32(u[i])));
    } else {
      const float gv = g[i];
      const float sg = 1.f / (1.f + expf(-gv));
      h[i] = (gv * sg) * u[i];
    }
  }
}

hipError_t launch_silu_mul(const void *g, const void *u, void *h, int64_t n, bool f32, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536;
  if (f32)
    hipLaunchKernelGGL(silu_mul_kernel<float>, dim3(blocks), dim3(256), 0, st, (const float *)g, (const float *)u,
                       (float *)h, n);
  else
    hipLaunchKernelGGL(silu_mul_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)g,
                       (const uint16_t *)u, (uint16_t *)h, n);
  return hipGetLastError();
}

hipError_t launch_qmv_generic(const QmmArgs &a, hipStream_t st) {
  dim3 grid(a.N, a.M);
  if (a.mode == MXFP8) {
    if (a.x_f32)
      hipLaunchKernelGGL((qmv_generic_kernel<MXFP8, true>), grid, dim3(64), 0, st, a.x, a.w, a.s, a.y, a.M, a.N, a.K);
    else
      hipLaunchKernelGGL((qmv_generic_kernel<MXFP8, false>), grid, dim3(64), 0, st, a.x, a.w, a.s, a.y, a.M, a.N, a.K);
  } else {
    if (a.x_f32)
      hipLaunchKernelGGL((qmv_generic_kernel<NVFP4, true>), grid, dim3(64), 0, st, a.x, a.w, a.s, a.y, a.M, a.N, a.K);
    else
      hipLaunchKernelGGL((qmv_generic_kernel<NVFP4, false>), grid, dim3(64), 0, st, a.x, a.w, a.s, a.y, a.M, a.N, a.K);
  }
  return hipGetLastError();
}

}  // namespace qmm
