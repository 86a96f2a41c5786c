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
// one wave per (row, m), lanes stride elements; exact integer decoders.
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
    acc = __builtin_fmaf(xk, e * sc, acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if (XF32)
      ((float *)yv)[(int64_t)m * N + n] = acc;
    else
      ((uint16_t *)yv)[(int64_t)m * N + n] = f32_to_bf16_rne(acc);
  }
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
  if (a.mode == MXFP8) return a.x_f32 ? launch_qmv_mode<MXFP8, true>(a, st) : launch_qmv_mode<MXFP8, false>(a, st);
  return a.x_f32 ? launch_qmv_mode<NVFP4, true>(a, st) : launch_qmv_mode<NVFP4, false>(a, st);
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
