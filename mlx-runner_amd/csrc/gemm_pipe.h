// Pieces shared by the pipelined prefill GEMMs (mxfp8 on the scaled fp8 MFMA,
// nvfp4 on the bf16 MFMA): tile order, LDS DMA, barrier/wait helpers and the
// weight-scale repack.
#pragma once

#include "qmm_device.h"

namespace qmm {

// Tile order: the hardware hands workgroup b to XCD b % 8.  Each XCD gets a
// contiguous run of tile indices, and tiles are numbered in groups of 4 M-tiles
// walked down M first, so the ~32 blocks resident on one XCD cover a 4 x 8
// patch of (x rows, W rows) and share those operand slabs in that XCD's L2.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int *tm, int *tn) {
  const int T = tiles_m * tiles_n;
  const int base = T / 8, rem = T % 8;
  const int x = b % 8, local = b / 8;
  const int t = x * base + (x < rem ? x : rem) + local;
  constexpr int G = 4;
  const int group = t / (G * tiles_n);
  const int first_m = group * G;
  const int gm = (tiles_m - first_m) < G ? (tiles_m - first_m) : G;
  const int idx = t - group * G * tiles_n;
  *tm = first_m + idx % gm;
  *tn = idx / gm;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// LDS DMA: lane i's 16 (4) bytes at g land at LDS byte l + 16 i (4 i); l must be
// wave-uniform.  Issued from assembly so that the compiler inserts no waits of
// its own for it: every user waits explicitly with s_waitcnt vmcnt.
__device__ __forceinline__ void gp_dma16(const void *g, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(l), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void gp_dma4(const void *g, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(l), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory operations are in flight and
// its LDS reads are done, then barrier the workgroup.
template <int N>
__device__ __forceinline__ void gp_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void gp_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void gp_barrier_only() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// Weight scales [N, nb bytes] (row-major, as loaded) -> tile-major: for each
// 256-row tile and each dword column d of the rows, 256 contiguous dwords (one
// per row): out[((tile * (nb / 4) + d) * 256 + r % 256] = row r's dword d.  A
// thread reads CH consecutive dwords of one row; rows past N (up to the next
// multiple of 256) repeat row N - 1.  Consecutive threads take consecutive rows,
// so every write is coalesced.
template <int CH>
__global__ __launch_bounds__(256) void repack_scales_kernel(const uint8_t *__restrict__ s, int64_t N, int nb,
                                                            uint32_t *__restrict__ out) {
  const int dpr = nb >> 2, chunks = dpr / CH;  // host: dpr % CH == 0
  const int64_t total = ((N + 255) >> 8) * chunks * 256;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rr = i & 255, tc = i >> 8;
    const int64_t tile = tc / chunks, c = tc % chunks;
    const int64_t r = min(tile * 256 + rr, N - 1);
    const uint8_t *src = s + r * nb + 4 * CH * c;
    uint32_t d[CH];
    if constexpr (CH == 4) {
      const uint4 u = *(const uint4 *)src;
      d[0] = u.x, d[1] = u.y, d[2] = u.z, d[3] = u.w;
    } else {
      d[0] = *(const uint32_t *)src;
    }
#pragma unroll
    for (int k = 0; k < CH; ++k) out[((tile * dpr + CH * c + k) << 8) + rr] = d[k];
  }
}

// Host: launch the repack (16-byte reads when the rows allow it); declared in qmm_launch.h.

}  // namespace qmm
