// Dequantize (mlx_dequantize, src/mlx.zig:274) and quantize (mlx_quantize,
// src/mlx.zig:278) for the mxfp8 / nvfp4 layouts.
//
// dequant: one thread per packed uint32 word (4 mxfp8 / 8 nvfp4 elements).
// Elements go through the same gfx950 converters the matmul kernels use, so the
// exhaustive dequant test pins the in-kernel unpack as well; the product with
// the group scale is one f32 multiply (exact for every finite in-range value).
//
// quantize: one thread per group.  Every rounding decision is an exact
// comparison (see the rule in qmm.h), so the result is bit-identical to the
// CPU restatement.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

template <int MODE, bool OUT_F32>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *__restrict__ w, const uint8_t *__restrict__ s,
                                                      void *__restrict__ out, int64_t N, int64_t K) {
  const int64_t epw = (MODE == MXFP8) ? 4 : 8;
  const int64_t wpr = K / epw;
  const int64_t total = N * wpr;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / wpr, wi = i % wpr;
    const int64_t k0 = wi * epw;
    const uint32_t word = w[i];
    float v[8];
    if constexpr (MODE == MXFP8) {
      const float sc = e8m0_to_f32(s[n * (K / 32) + k0 / 32]);
      f32x2_t a = fp8x2_to_f32x2<false>(word), b = fp8x2_to_f32x2<true>(word);
      v[0] = a.x * sc; v[1] = a.y * sc; v[2] = b.x * sc; v[3] = b.y * sc;
    } else {
      const float sc = __builtin_amdgcn_cvt_f32_fp8((int)s[n * (K / 16) + k0 / 16], 0);
      f32x2_t a = fp4x2_to_f32x2<0>(word), b = fp4x2_to_f32x2<1>(word);
      f32x2_t c = fp4x2_to_f32x2<2>(word), d = fp4x2_to_f32x2<3>(word);
      v[0] = a.x * sc; v[1] = a.y * sc; v[2] = b.x * sc; v[3] = b.y * sc;
      v[4] = c.x * sc; v[5] = c.y * sc; v[6] = d.x * sc; v[7] = d.y * sc;
    }
    if constexpr (OUT_F32) {
      float *o = (float *)out + n * K + k0;
#pragma unroll
      for (int j = 0; j < (int)epw; ++j) o[j] = v[j];
    } else {
      uint16_t *o = (uint16_t *)out + n * K + k0;
#pragma unroll
      for (int j = 0; j < (int)epw; ++j) o[j] = f32_to_bf16_rne(v[j]);
    }
  }
}

hipError_t launch_dequant(int mode, const uint8_t *w, const uint8_t *s, int64_t N, int64_t K, void *out,
                          bool out_f32, hipStream_t st) {
  const int64_t words = N * (mode == MXFP8 ? K / 4 : K / 8);
  if (words == 0) return hipSuccess;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  const uint32_t *wp = (const uint32_t *)w;
  if (mode == MXFP8) {
    if (out_f32)
      hipLaunchKernelGGL((dequant_kernel<MXFP8, true>), dim3(blocks), dim3(256), 0, st, wp, s, out, N, K);
    else
      hipLaunchKernelGGL((dequant_kernel<MXFP8, false>), dim3(blocks), dim3(256), 0, st, wp, s, out, N, K);
  } else {
    if (out_f32)
      hipLaunchKernelGGL((dequant_kernel<NVFP4, true>), dim3(blocks), dim3(256), 0, st, wp, s, out, N, K);
    else
      hipLaunchKernelGGL((dequant_kernel<NVFP4, false>), dim3(blocks), dim3(256), 0, st, wp, s, out, N, K);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- quantize

// Nearest E4M3 code to v >= 0 (finite), ties to even, saturating at 448.
__device__ __forceinline__ uint32_t e4m3_code_rne_sat(float v) {
  if (!(v > 0.f)) return 0u;
  if (v >= 448.f) return 0x7Eu;
  int e = (int)((__float_as_uint(v) >> 23) & 0xFF) - 127;  // floor(log2 v) for normal v
  if (v < 0x1p-126f) e = -127;                            // f32 subnormal: far below the e4m3 range
  int q = e - 3;
  if (q < -9) q = -9;
  float r = __builtin_rintf(__builtin_ldexpf(v, -q));  // exact scaling, RNE
  r = __builtin_ldexpf(r, q);
  if (r > 448.f) r = 448.f;
  if (r < 0x1p-6f) return (uint32_t)__builtin_ldexpf(r, 9);  // subnormal m/8 * 2^-6
  uint32_t u = __float_as_uint(r);
  uint32_t E = ((u >> 23) & 0xFF) - 127 + 7;
  uint32_t Mt = (u >> 20) & 7u;
  return (E << 3) | Mt;
}

__device__ __forceinline__ float load_in(const void *in, bool f32, int64_t i) {
  return f32 ? ((const float *)in)[i] : bf16_to_f32(((const uint16_t *)in)[i]);
}

template <int MODE>
__global__ __launch_bounds__(256) void quantize_kernel(const void *__restrict__ in, bool in_f32, int64_t N, int64_t K,
                                                       uint32_t *__restrict__ wq, uint8_t *__restrict__ s) {
  constexpr int G = (MODE == MXFP8) ? 32 : 16;
  const int64_t gpr = K / G;
  const int64_t total = N * gpr;
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < total; gi += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = gi / gpr, g = gi % gpr;
    const int64_t base = n * K + g * G;
    float v[G];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      v[i] = load_in(in, in_f32, base + i);
      amax = fmaxf(amax, fabsf(v[i]));
    }
    if constexpr (MODE == MXFP8) {
      int X;
      if (amax == 0.f) {
        X = 0;
      } else {
        uint32_t u = __float_as_uint(amax);
        int e = (int)((u >> 23) & 0xFF);
        int fl = e - 127;                                          // floor(log2 amax)
        if (e == 0) fl = 31 - __builtin_clz(u & 0x7FFFFF) - 149;  // f32 subnormal amax
        X = fl - 8 + 127;
        X = X < 0 ? 0 : (X > 254 ? 254 : X);
      }
      s[gi] = (uint8_t)X;
      // elements: v / 2^(X-127), exact for every value that can round to a nonzero code
      const int sh = 127 - X;
      uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < G; ++i) {
        float p = __builtin_ldexpf(v[i], sh);
        uint32_t c = e4m3_code_rne_sat(fabsf(p));
        if (signbit(p) && c != 0u) c |= 0x80u;
        words[i >> 2] |= c << (8 * (i & 3));
      }
      uint32_t *o = wq + n * (K / 4) + g * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = words[j];
    } else {
      // scale: the E4M3 code nearest to amax/6 (ties to even), decided exactly in double
      uint32_t best = 0u;
      if (amax > 0.f) {
        uint32_t c0 = e4m3_code_rne_sat(amax / 6.f);
        double bestd = -1.0;
        for (int d = -1; d <= 1; ++d) {
          int c = (int)c0 + d;
          if (c < 0 || c > 0x7E) continue;
          double cv = (double)e4m3_to_f32_int((uint32_t)c);
          double diff = fabs(6.0 * cv - (double)amax);
          if (bestd < 0.0 || diff < bestd || (diff == bestd && ((c & 1) == 0))) {
            bestd = diff;
            best = (uint32_t)c;
          }
        }
      }
      s[gi] = (uint8_t)best;
      const float sc = e4m3_to_f32_int(best);
      const float mids[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
      uint32_t words[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < G; ++i) {
        uint32_t c = 0u;
        if (sc != 0.f) {
          float ax = fabsf(v[i]);
          int ci = 0;
          bool odd_tie = false;  // ax sits exactly on the midpoint above an odd code
#pragma unroll
          for (int t = 0; t < 7; ++t) {
            ci += (ax > mids[t] * sc) ? 1 : 0;
            odd_tie |= (ax == mids[t] * sc) && (t & 1);
          }
          if (odd_tie) ci += 1;
          c = (uint32_t)ci;
          if (signbit(v[i]) && c != 0u) c |= 0x8u;
        }
        words[i >> 3] |= c << (4 * (i & 7));
      }
      uint32_t *o = wq + n * (K / 8) + g * 2;
      o[0] = words[0];
      o[1] = words[1];
    }
  }
}

hipError_t launch_quantize(int mode, const void *in, bool in_f32, int64_t N, int64_t K, uint32_t *wq, uint8_t *s,
                           hipStream_t st) {
  const int64_t groups = N * (K / (mode == MXFP8 ? 32 : 16));
  if (groups == 0) return hipSuccess;
  int64_t blocks = (groups + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (mode == MXFP8)
    hipLaunchKernelGGL((quantize_kernel<MXFP8>), dim3(blocks), dim3(256), 0, st, in, in_f32, N, K, wq, s);
  else
    hipLaunchKernelGGL((quantize_kernel<NVFP4>), dim3(blocks), dim3(256), 0, st, in, in_f32, N, K, wq, s);
  return hipGetLastError();
}

__global__ void fill_zero_bytes_kernel(uint8_t *__restrict__ p, int64_t n) {
  if ((int64_t)threadIdx.x < n) p[threadIdx.x] = 0;
}

// Zero-fill (a kernel rather than hipMemsetAsync, so the op stays safe to
// record into a HIP graph).
__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t *__restrict__ p, int64_t words) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t st) {
  const int64_t words = (int64_t)(bytes / 4);
  if (words > 0) {
    int64_t blocks = (words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, st, (uint32_t *)p, words);
  }
  if (bytes % 4) {
    // trailing bytes (odd-sized bf16 outputs): one more word-aligned store is not
    // possible without overrunning, so clear them with a byte kernel
    hipLaunchKernelGGL(fill_zero_bytes_kernel, dim3(1), dim3(64), 0, st, (uint8_t *)p + words * 4,
                       (int64_t)(bytes % 4));
  }
  return hipGetLastError();
}

int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const bool slot = dev >= 0 && dev < 64;
  if (slot) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  if (slot) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

hipError_t ensure_dynamic_lds(std::atomic<uint64_t> &done, const void *kernel, int bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

}  // namespace qmm
