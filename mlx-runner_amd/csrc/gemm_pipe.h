// Pieces shared by the pipelined prefill GEMMs (mxfp8 on the scaled fp8 MFMA,
// nvfp4 on the bf16 MFMA): tile order, LDS DMA, barrier/wait helpers and the
// weight-scale repack.
#pragma once

#include "qmm_device.h"
#include "qmm_launch.h"

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
// The same with the source as a wave-uniform base (SGPRs) plus a 32-bit lane offset.
__device__ __forceinline__ void gp_dma16s(const void *base, uint32_t off, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(off), "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void gp_dma4s(const void *base, uint32_t off, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(l), "v"(off), "s"(base)
               : "memory", "m0");
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

// Whether the output parts take 16-byte stores of 8 columns: every part's row length a
// multiple of 8 (so no 8-column piece crosses a part boundary) and every part 16-byte aligned.
__device__ __forceinline__ bool yout_vec(const YOut yo) {
  return ((yo.n0 | yo.n1 | yo.n2 | yo.n3) & 7) == 0 &&
         (((uintptr_t)yo.y0 | (uintptr_t)yo.y1 | (uintptr_t)yo.y2 | (uintptr_t)yo.y3) & 15) == 0;
}

// Epilogue of a wave's FI x FJ grid of 32x32 f32 accumulators (rows row0 + [0, 32 FI),
// cols col0 + [0, 32 FJ) of y[M, N], whose column c is column c - lo of part yo.at's part
// (one part: y itself); columns from col_end on are not this call's), bf16
// out, accumulator blocks i in [I0, I0 + NI).  Element v of lane l of a 32x32 block is
// row 8 (v / 4) + 4 (l / 32) + v % 4, col l % 32: a store straight from it writes two
// bytes per lane.  Instead each lane converts its rows 2u, 2u + 1 with one packed RNE
// conversion (bit-identical to f32_to_bf16_rne on every finite input; a NaN stays a NaN
// but keeps its sign), swaps the dword with its neighbour lane (DPP) and keeps one row
// of the two columns (v_perm: the even lane row 2u, the odd lane row 2u + 1), writes
// it to the wave's LDS region and reads the region back 16 bytes per lane along rows,
// so every global store writes 16 contiguous bytes (vec: yout_vec; otherwise, and at the
// last columns, element stores).  The region,
// (32 NI) x (64 FJ + 32) bytes, belongs to this wave; the caller guarantees that no
// other wave reads or writes it meanwhile.
typedef __bf16 gp_bf16x2_t __attribute__((ext_vector_type(2)));
template <int FI, int FJ, int I0, int NI>
__device__ __forceinline__ void gp_store_tile_bf16(const f32x16_t (&acc)[FI][FJ], uint8_t *region, int lane,
                                                   const YOut yo, int M, int row0, int col0, int col_end,
                                                   bool vec) {
  constexpr int PITCH = 64 * FJ + 32;  // bytes per region row (the pad spreads a write's rows over the banks)
  const int c = lane & 31, h = lane >> 5;
  const bool odd = c & 1;
  // v_perm selector over {neighbour's dword, own dword} (own bytes 0-3, neighbour's 4-7):
  // even lane: own low half, neighbour's low half (row 2u, columns c, c + 1);
  // odd lane: neighbour's high half, own high half (row 2u + 1, columns c - 1, c)
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        gp_bf16x2_t w;
        w[0] = (__bf16)acc[I0 + i][j][2 * u];
        w[1] = (__bf16)acc[I0 + i][j][2 * u + 1];
        const uint32_t own = __builtin_bit_cast(uint32_t, w);
        const uint32_t nb = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0xB1, 0xF, 0xF, true);  // lane ^ 1
        const uint32_t word = __builtin_amdgcn_perm(nb, own, sel);
        const int row = i * 32 + 8 * (u >> 1) + 4 * h + 2 * (u & 1) + (odd ? 1 : 0);
        *(uint32_t *)(region + row * PITCH + (j * 32 + (c & ~1)) * 2) = word;
      }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int LPR = FJ * 4;    // lanes per row (16-byte pieces)
  constexpr int RPI = 64 / LPR;  // rows per instruction
  if (vec && row0 + (I0 + NI) * 32 <= M && col0 + FJ * 32 <= col_end) {  // the whole block is inside
#pragma unroll
    for (int it = 0; it < NI * 32 / RPI; ++it) {
      const int row = it * RPI + lane / LPR, piece = lane % LPR;
      const uint4 d = *(const uint4 *)(region + row * PITCH + piece * 16);
      *(uint4 *)yo.at(row0 + I0 * 32 + row, col0 + piece * 8) = d;
    }
    return;
  }
#pragma unroll
  for (int it = 0; it < NI * 32 / RPI; ++it) {
    const int row = it * RPI + lane / LPR, piece = lane % LPR;
    const uint4 d = *(const uint4 *)(region + row * PITCH + piece * 16);
    const int gr = row0 + I0 * 32 + row, gc = col0 + piece * 8;
    if (gr < M) {
      if (vec && gc + 8 <= col_end) {
        *(uint4 *)yo.at(gr, gc) = d;
      } else {
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (gc + e < col_end) *yo.at(gr, gc + e) = (uint16_t)(dw[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

// Split tiles (a tile's K steps run by S blocks): each block stores its wave's FI x FJ
// fp32 accumulators as they sit in the registers, the float4 of elements 4 v4 .. 4 v4 + 3
// of accumulator (i, j) of lane l at ((wave * FI * FJ + i * FJ + j) * 4 + v4) * 64 + l of
// the block's slot (8 waves: 8 * FI * FJ * 1 KiB per slot).  Accumulator rows i with
// 32 i >= live_rows (the wave's rows past the last x row: padding of a short x) are
// neither stored nor summed.
template <int FI, int FJ>
__device__ __forceinline__ void gp_store_partial(const f32x16_t (&acc)[FI][FJ], float *__restrict__ slot, int wave,
                                                 int lane, int live_rows) {
  float4 *pw = (float4 *)slot + (size_t)wave * FI * FJ * 4 * 64 + lane;
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    if (32 * i >= live_rows) break;
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4)
        pw[((i * FJ + j) * 4 + v4) * 64] =
            make_float4(acc[i][j][4 * v4], acc[i][j][4 * v4 + 1], acc[i][j][4 * v4 + 2], acc[i][j][4 * v4 + 3]);
  }
}

// The split-tile reduce, one thread per float4 of the partial layout: float4 (wave, q, lane)
// of split tile t, q = (i FJ + j) 4 + v4, is summed over the tile's S <= GP_MAX_SPLIT slots
// (t S .. t S + S - 1) in K order, the same order whichever block finished first, so the
// result is deterministic.  Its four values are rows 32 i + 8 v4 + 4 (lane / 32) + [0, 4),
// column 32 j + lane % 32 of the wave's region at (row0, col0) of y (yo.at); they are rounded to bf16
// as the tile epilogue rounds (rows from M on and columns from col_end on are not stored).
// All S loads are issued before the first add, so a thread waits for one round trip, not S.
constexpr int GP_MAX_SPLIT = 8;
template <int FI, int FJ>
__device__ __forceinline__ void gp_reduce_quad(const float *__restrict__ part, const YOut yo, int M, int col_end,
                                               int t, int S, int wave, int q, int lane, int row0, int col0) {
  const int i = q / (FJ * 4), j = (q / 4) % FJ, v4 = q % 4;
  const int r = row0 + 32 * i + 8 * v4 + 4 * (lane >> 5), c = col0 + 32 * j + (lane & 31);
  if (r >= M || c >= col_end) return;  // not stored by the split blocks either (rows past M)
  const float4 *pw = (const float4 *)part + ((size_t)t * S * 8 + wave) * FI * FJ * 4 * 64 + q * 64 + lane;
  const size_t slot = (size_t)8 * FI * FJ * 4 * 64;  // float4s per slot
  float4 f[GP_MAX_SPLIT];
#pragma unroll
  for (int k = 0; k < GP_MAX_SPLIT; ++k) f[k] = pw[(k < S ? k : S - 1) * slot];
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < GP_MAX_SPLIT; ++k)
    if (k < S) s.x += f[k].x, s.y += f[k].y, s.z += f[k].z, s.w += f[k].w;
  const float v[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (r + e < M) *yo.at(r + e, c) = __builtin_bit_cast(uint16_t, (__bf16)v[e]);
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
