// Prefill quantized matmul (M > 8) and the dense bf16 linear fallback.
//
// y[M, N] = x[M, K] @ deq(W)[N, K].T for the prefill chunks mlx-runner feeds
// through the same qmm call sites (src/engine.zig:364-382, M <= 2048 per chunk),
// and y = x @ W.T for dense bf16 weights (linear, src/model.zig:200-211).
//
// Tiling (gfx950, wave64, 256 threads):
//   block tile 128 (x rows) x 128 (W rows), K step 32;
//   each thread stages 16 elements of one x row and 16 of one W row into LDS;
//   W elements are unpacked with the gfx950 converters, so LDS holds bf16:
//     nvfp4: E2M1 times its E4M3 scale in f32, exact in bf16 (at most 6
//            significant bits, magnitudes 2^-10 .. 2688);
//     mxfp8: the E4M3 codes unscaled (exact in bf16).  A K step is one 32-element
//            scale block, so each step's MFMA sums go to a temporary and are added
//            to the accumulator times the W row's E8M0 scale in f32: a weight whose
//            f32 (or bf16) dequant would overflow or underflow still multiplies x
//            as its true value, as in the other kernels;
//   4 waves in 2x2, each owning 64x64 of the tile as 2x2 v_mfma_f32_32x32x16_bf16
//   accumulators (fp32); epilogue rounds to bf16 (RNE).
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

constexpr int DENSE_BF16 = 2;

namespace {
constexpr int BM = 128, BN = 128, BK = 32, LDK = BK + 8;  // LDS row pitch (bf16), 80 bytes
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
}

// 16 consecutive W elements of row n starting at k (k a multiple of 16) as 8 bf16 pairs
// (mxfp8: unscaled codes, the block's scale in *sc_out; otherwise dequantized).
template <int MODE>
__device__ __forceinline__ void load_w16(const uint8_t *__restrict__ w, const uint8_t *__restrict__ s, int64_t n,
                                         int k, int K, uint32_t out[8], float *sc_out) {
  if constexpr (MODE == MXFP8) {
    const uint4 q = *(const uint4 *)(w + n * (int64_t)K + k);
    *sc_out = e8m0_to_f32(s[n * (int64_t)(K >> 5) + (k >> 5)]);
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(d[j]));
      out[2 * j + 1] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(d[j]));
    }
  } else if constexpr (MODE == NVFP4) {
    const uint2 q = *(const uint2 *)(w + n * (int64_t)(K >> 1) + (k >> 1));
    const float sc = __builtin_amdgcn_cvt_f32_fp8((int)s[n * (int64_t)(K >> 4) + (k >> 4)], 0);
    const uint32_t d[2] = {q.x, q.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x2_t a = fp4x2_to_f32x2<0>(d[j]), b = fp4x2_to_f32x2<1>(d[j]);
      f32x2_t c = fp4x2_to_f32x2<2>(d[j]), e = fp4x2_to_f32x2<3>(d[j]);
      out[4 * j + 0] = pack_bf16x2(a.x * sc, a.y * sc);
      out[4 * j + 1] = pack_bf16x2(b.x * sc, b.y * sc);
      out[4 * j + 2] = pack_bf16x2(c.x * sc, c.y * sc);
      out[4 * j + 3] = pack_bf16x2(e.x * sc, e.y * sc);
    }
  } else {
    const uint16_t *wr = (const uint16_t *)w + n * (int64_t)K + k;
    const uint4 a = ((const uint4 *)wr)[0], b = ((const uint4 *)wr)[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint16_t *__restrict__ x, const uint8_t *__restrict__ w,
                                                        const uint8_t *__restrict__ s, uint16_t *__restrict__ y, int M,
                                                        int N, int K) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDK];
  __shared__ float Ss[MODE == MXFP8 ? BN : 1];  // mxfp8: the step's scale of each W row
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int lrow = tid >> 1, lh = tid & 1;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  for (int k0 = 0; k0 < K; k0 += BK) {
    const int kk = k0 + 16 * lh;
    uint4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
    const int m = m0 + lrow;
    if (m < M && kk < K) {
      const uint4 *p = (const uint4 *)(x + (int64_t)m * K + kk);
      a0 = p[0];
      a1 = p[1];
    }
    uint32_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sc = 0.f;
    const int n = n0 + lrow;
    if (n < N && kk < K) load_w16<MODE>(w, s, n, kk, K, b, &sc);
    uint4 *ad = (uint4 *)(As + lrow * LDK + 16 * lh);
    ad[0] = a0;
    ad[1] = a1;
    uint4 *bd = (uint4 *)(Bs + lrow * LDK + 16 * lh);
    bd[0] = make_uint4(b[0], b[1], b[2], b[3]);
    bd[1] = make_uint4(b[4], b[5], b[6], b[7]);
    if constexpr (MODE == MXFP8)
      if (lh == 0) Ss[lrow] = sc;  // both halves of a row's step are one 32-block
    __syncthreads();
    f32x16_t part[2][2];
    if constexpr (MODE == MXFP8) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) part[i][j][v] = 0.f;
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      bf16x8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const bf16x8_t *)(As + (wm * 64 + i * 32 + (lane & 31)) * LDK + kh * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *(const bf16x8_t *)(Bs + (wn * 64 + j * 32 + (lane & 31)) * LDK + kh * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (MODE == MXFP8)
            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], part[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
    if constexpr (MODE == MXFP8) {
      // accumulator column = W row wn * 64 + j * 32 + lane % 32 of the tile
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float scj = Ss[wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[i][j][v] = __builtin_fmaf(part[i][j][v], scj, acc[i][j][v]);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (row < M && col < N) y[(int64_t)row * N + col] = f32_to_bf16_rne(acc[i][j][v]);
      }
    }
}

bool gemm_ok(const QmmArgs &a) {
  // bf16 x; K a multiple of 16 (one nvfp4 group / half an mxfp8 group per loader).
  return !a.x_f32 && a.K % 16 == 0 && a.M > 0 && a.N > 0 && (a.mode != MXFP8 || a.K % 32 == 0);
}

hipError_t launch_gemm(const QmmArgs &a, hipStream_t st) {
  if (!gemm_ok(a)) return hipErrorInvalidValue;
  dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  if (a.mode == MXFP8)
    hipLaunchKernelGGL((gemm_bf16_kernel<MXFP8>), grid, dim3(256), 0, st, (const uint16_t *)a.x, a.w, a.s,
                       (uint16_t *)a.y, a.M, a.N, a.K);
  else
    hipLaunchKernelGGL((gemm_bf16_kernel<NVFP4>), grid, dim3(256), 0, st, (const uint16_t *)a.x, a.w, a.s,
                       (uint16_t *)a.y, a.M, a.N, a.K);
  return hipGetLastError();
}

// ---------------------------------------------------------------- dense bf16 linear

// M <= 8: one wave per 4 W rows, lanes over 16-byte (8-element) chunks.
template <int M>
__global__ __launch_bounds__(64) void gemv_bf16_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ w,
                                                       uint16_t *__restrict__ y, int N, int K) {
  constexpr int R = 4;
  const int lane = threadIdx.x;
  const int n0 = blockIdx.x * R;
  const int C = K >> 3;
  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  for (int c = lane; c < C; c += 64) {
    uint4 q[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = n0 + r < N ? n0 + r : N - 1;
      q[r] = load_stream16((const uint4 *)(w + (int64_t)n * K) + c);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 xv = ((const uint4 *)(x + (int64_t)m * K))[c];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float t = acc[r][m];
        t = dot2_bf16(__builtin_bit_cast(bf16x2_t, q[r].x), xv.x, t);
        t = dot2_bf16(__builtin_bit_cast(bf16x2_t, q[r].y), xv.y, t);
        t = dot2_bf16(__builtin_bit_cast(bf16x2_t, q[r].z), xv.z, t);
        t = dot2_bf16(__builtin_bit_cast(bf16x2_t, q[r].w), xv.w, t);
        acc[r][m] = t;
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
    const int r = lane / M, m = lane % M;
    if (n0 + r < N) y[(int64_t)m * N + n0 + r] = f32_to_bf16_rne(out);
  }
}

hipError_t launch_linear_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y, int M, int N, int K,
                              hipStream_t st) {
  if (K % 16 != 0 || M <= 0 || N <= 0) return hipErrorInvalidValue;
  if (M <= 8) {
    dim3 grid((N + 3) / 4);
    switch (M) {
#define QMM_GEMV_CASE(MM) \
  case MM: hipLaunchKernelGGL((gemv_bf16_kernel<MM>), grid, dim3(64), 0, st, x, w, y, N, K); break;
      QMM_GEMV_CASE(1) QMM_GEMV_CASE(2) QMM_GEMV_CASE(3) QMM_GEMV_CASE(4)
      QMM_GEMV_CASE(5) QMM_GEMV_CASE(6) QMM_GEMV_CASE(7) QMM_GEMV_CASE(8)
#undef QMM_GEMV_CASE
    }
    return hipGetLastError();
  }
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_bf16_kernel<DENSE_BF16>), grid, dim3(256), 0, st, x, (const uint8_t *)w, nullptr, y, M,
                     N, K);
  return hipGetLastError();
}

}  // namespace qmm
