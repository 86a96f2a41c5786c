// Chunked (matrix) form of the gated-delta recurrence for long T (prefill), on
// the f32 MFMA.  Same results as the step-by-step kernel in gdn.hip (to f32
// rounding): for each (b, value head hv, key head hk = hv / (Hv / Hk)) and
// chunk of C steps t = 0..C-1 with S0 the state before the chunk,
//   G_t = sum_{i <= t} log g_i (f64),  D_tj = exp(G_t - G_j) for j <= t,
//   gam_t = exp(G_t),  tail_t = exp(G_{C-1} - G_t),
//   A   = (I + tril(diag(beta) (D o K K^T), -1))^-1,  Ap = A diag(beta),
//   M   = tril(D o Q K^T)  (diagonal included),
//   U   = V - (gam o K) S0^T                         [C, Dv]
//   Dl  = Ap U                                       [C, Dv]  (the chunk's deltas)
//   Y   = (gam o Q) S0^T + M Dl                      [C, Dv]
//   S1  = gam_{C-1} S0 + Dl^T (tail o K)             [Dv, Dk]
// which unrolls S_t = g_t S_{t-1} + dlt_t k_t^T, dlt_t = beta_t (v_t - g_t S_{t-1} k_t),
// y_t = S_t q_t over the chunk.  Steps past T are padded with g = 1, beta = 0
// and zero q, k, v: they leave the state as it is and write nothing.
//
// gdn_chunk_prep, one workgroup per (b, hv, chunk), every chunk in parallel:
// K K^T and Q K^T on the MFMA, A by blocks (16 x 16 diagonal blocks by forward
// substitution, the blocks below by MFMA products, one block diagonal at a
// time), and Ap, M, gam, tail into a workspace.
// gdn_chunk_scan, one workgroup per (b, hv, 16 state rows): the chunks in
// order; the rows' state stays in MFMA accumulators (wave w holds columns
// 32 w .. 32 w + 31), and per chunk the products above run as 16 x 16 MFMA tiles.
#include <mutex>
#include <type_traits>

#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

constexpr int GC = 64;    // steps per chunk
constexpr int GDK = 128;  // key head dim
constexpr int GR = 16;    // state rows per scan workgroup
constexpr int KP = GDK + 4;  // LDS row pitch of [.][GDK] arrays (floats)
constexpr int TP = GC + 4;   // LDS row pitch of [.][GC] arrays (16-byte aligned rows for float4 runs)

// workspace per (b, hv, chunk), in floats: Ap and M (the 16 x 16 blocks on and below the
// diagonal; blocks above it are read from one shared zero block at the end), gam, tail
constexpr int WS_AP = 0;
constexpr int WS_M = WS_AP + GC * GC;
constexpr int WS_GAM = WS_M + GC * GC;
constexpr int WS_TAIL = WS_GAM + GC;
constexpr int WS_CHUNK = WS_TAIL + GC;
constexpr int WS_ZERO = 64;  // the zero block's floats

// Scan workgroup -> (b * Hv + hv, first state row).  Workgroups are dealt to the 8 XCDs in
// turn (blockIdx % 8).  Those that read the same key head's q and k (Hv / Hk value heads x
// Dv / 16 row groups) have consecutive linear indices, and each XCD takes a contiguous range
// of them, so a key head's chunks are fetched into one XCD's L2 (and a value head's Ap, M
// too).  False for the grid's padding workgroups (the grid is a multiple of 8).
__device__ __forceinline__ bool scan_wg(int nwg, int nrg, int &nh, int &r0) {
  const int per = (nwg + 7) / 8;
  const int L = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (L >= nwg) return false;
  nh = L / nrg;
  r0 = (L - nh * nrg) * GR;
  return true;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// D += A B for one 16 x 16 tile over K = 4 NK, lane group g = l / 16 taking k = NK g + m
// (m < NK), from operands in registers.  v_mfma_f32_16x16x4f32 takes A(l % 16, k) and
// B(k, l % 16) from lane l for the k of its lane group, and the order of the terms of a
// sum is free, so lane l supplies a[m] = A(l % 16, NK g + m) and b[m] = B(NK g + m, l % 16):
// runs of NK consecutive elements of a row of A and a column of B.  Output element v of
// lane l is D(4 (l / 16) + v, l % 16).
template <int NK>
__device__ __forceinline__ f32x4 mm_rr(f32x4 c, const float *a, const float *b) {
#pragma unroll
  for (int m = 0; m < NK; ++m) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m], b[m], c, 0, 0, 0);
  return c;
}

// As mm_rr on the bf16 MFMA (v_mfma_f32_16x16x32_bf16), 8 k per lane per instruction:
// element e of a[m] and of b[m] in lane l pair up, whatever k they stand for.
template <int NK>
__device__ __forceinline__ f32x4 mm_bf(f32x4 c, const bf16x8_t *a, const bf16x8_t *b) {
#pragma unroll
  for (int m = 0; m < NK; ++m) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[m], b[m], c, 0, 0, 0);
  return c;
}

// NK consecutive floats of LDS (16-byte aligned) into registers
template <int NK>
__device__ __forceinline__ void lds_run(float *o, const float *p) {
#pragma unroll
  for (int m = 0; m < NK; m += 4) *(float4 *)&o[m] = *(const float4 *)(p + m);
}

// 8 consecutive elements of a bf16 or f32 array as f32
template <bool F32>
__device__ __forceinline__ void ld8f(const void *p, int64_t i, float *o) {
  if constexpr (F32) {
    const float4 a = ((const float4 *)((const float *)p + i))[0], b = ((const float4 *)((const float *)p + i))[1];
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  } else {
    const uint4 a = *(const uint4 *)((const uint16_t *)p + i);
    const uint32_t wv[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = __uint_as_float(wv[j] << 16);
      o[2 * j + 1] = __uint_as_float(wv[j] & 0xFFFF0000u);
    }
  }
}

template <bool F32>
__device__ __forceinline__ float ld1f(const void *p, int64_t i) {
  if constexpr (F32)
    return ((const float *)p)[i];
  else
    return bf16_to_f32(((const uint16_t *)p)[i]);
}

// e^x from an f64 argument: 2^(x log2 e) split into an integer and a fraction in [0, 1);
// the fraction's power on v_exp_f32, the integer on the exponent (underflow gives 0)
__device__ __forceinline__ float exp_f64arg(double x) {
  const double yv = x * 1.4426950408889634;  // log2(e)
  const double fl = floor(yv);
  const float f = (float)(yv - fl);
  const double cl = fl < -400.0 ? -400.0 : fl;
  return __builtin_ldexpf(__builtin_amdgcn_exp2f(f), (int)cl);
}

// LDS (floats): lm (L, strictly lower), ai (A) [GC][TP]; bt [GC]; gd (doubles) [GC]
constexpr size_t PREP_LDS = (size_t)(2 * GC * TP + GC) * 4 + GC * 8;

template <bool IN_F32>
__global__ __launch_bounds__(256) void gdn_chunk_prep(const void *__restrict__ q, const void *__restrict__ k,
                                                      const float *__restrict__ g, const void *__restrict__ beta,
                                                      int beta_f32, float *__restrict__ ws, int T, int Hk, int Hv,
                                                      int nch) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *lm = lds, *ai = lm + GC * TP, *bt = ai + GC * TP;
  double *gd = (double *)(bt + GC);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int ci = blockIdx.x % nch, nh = blockIdx.x / nch;  // nh = b * Hv + hv
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
  float *out = ws + ((int64_t)nh * nch + ci) * WS_CHUNK;

  if (wave == 0) {  // G_t: inclusive prefix sum of the log-decays over the wave, in f64
    double a = 0.0;
    float be = 0.f;
    if (lane < n) {
      const int64_t gi = ((int64_t)b * T + t0 + lane) * Hv + hv;
      const double gv = (double)g[gi];
      // g = 0 (either sign) wipes the state: exp of the difference underflows to 0.  A NaN or
      // negative g gives NaN from that step on, as the step kernel's multiply by g gives NaN
      // for a NaN g (a negative g, outside the model's (0, 1], has no logarithm).
      a = gv > 0.0 ? log(gv) : (gv == 0.0 ? -1.0e4 : __longlong_as_double(0x7FF8000000000000LL));
      be = beta_f32 ? ((const float *)beta)[gi] : bf16_to_f32(((const uint16_t *)beta)[gi]);
    }
#pragma unroll
    for (int o = 1; o < GC; o <<= 1) {
      const double x = __shfl_up(a, o);
      if (lane >= o) a += x;
    }
    gd[lane] = a;
    bt[lane] = be;
    const double gl = __shfl(a, GC - 1);
    out[WS_GAM + lane] = exp_f64arg(a);
    out[WS_TAIL + lane] = exp_f64arg(gl - a);
  }

  // K K^T and Q K^T for the 10 blocks (tb, jb), jb <= tb, block e = tb (tb + 1) / 2 + jb
  // on wave e % 4; operands are rows of K and Q straight from global memory (rows past
  // n read as zero)
  auto row_run = [&](const void *p, int t, float *o) __attribute__((always_inline)) {
    const int tt = t < n ? t : n - 1;
    const int64_t off = (((int64_t)b * T + t0 + tt) * Hk + hk) * GDK + 32 * lg;
#pragma unroll
    for (int u = 0; u < 4; ++u) ld8f<IN_F32>(p, off + 8 * u, o + 8 * u);
    if (t >= n) {
#pragma unroll
      for (int m = 0; m < 32; ++m) o[m] = 0.f;
    }
  };
  auto row_run_bf = [&](const void *p, int t, bf16x8_t *o) __attribute__((always_inline)) {
    const int tt = t < n ? t : n - 1;
    const bf16x8_t *src = (const bf16x8_t *)((const uint16_t *)p + (((int64_t)b * T + t0 + tt) * Hk + hk) * GDK + 32 * lg);
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = t < n ? src[u] : bf16x8_t{};
  };
  f32x4 kk[3], qk[3];
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    const int e = wave + 4 * s;
    if (e < 10) {
      const int tb = (e >= 1) + (e >= 3) + (e >= 6), jb = e - tb * (tb + 1) / 2;
      if constexpr (IN_F32) {
        float ka[32], qa[32], kb[32];
        row_run(k, 16 * tb + li, ka);
        row_run(q, 16 * tb + li, qa);
        row_run(k, 16 * jb + li, kb);
        kk[s] = mm_rr<32>(f32x4{0.f, 0.f, 0.f, 0.f}, ka, kb);
        qk[s] = mm_rr<32>(f32x4{0.f, 0.f, 0.f, 0.f}, qa, kb);
      } else {  // bf16 products are exact in f32: the bf16 MFMA, 32 k per instruction
        bf16x8_t ka[4], qa[4], kb[4];
        row_run_bf(k, 16 * tb + li, ka);
        row_run_bf(q, 16 * tb + li, qa);
        row_run_bf(k, 16 * jb + li, kb);
        kk[s] = mm_bf<4>(f32x4{0.f, 0.f, 0.f, 0.f}, ka, kb);
        qk[s] = mm_bf<4>(f32x4{0.f, 0.f, 0.f, 0.f}, qa, kb);
      }
    }
  }
  __syncthreads();  // gd, bt
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    const int e = wave + 4 * s;
    if (e < 10) {
      const int tb = (e >= 1) + (e >= 3) + (e >= 6), jb = e - tb * (tb + 1) / 2;
      const int j = 16 * jb + li;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 16 * tb + 4 * lg + v;
        const float d = j <= t ? exp_f64arg(gd[t] - gd[j]) : 0.f;
        if (j < t) lm[t * TP + j] = bt[t] * d * kk[s][v];
        out[WS_M + t * GC + j] = d * qk[s][v];
      }
    }
  }
  __syncthreads();  // lm

  // A = (I + L)^-1 by 16 x 16 blocks.  Diagonal block w on wave w, column li per lane:
  // x[t] = delta_t,li - sum_{j<t} L[t][j] x[j]; rows above li come out zero by themselves.
  {
    const float *lb = lm + 16 * wave * TP + 16 * wave;
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int j = 0; j < t; ++j) {
        if (j & 1)
          s1 = __builtin_fmaf(lb[t * TP + j], x[j], s1);
        else
          s0 = __builtin_fmaf(lb[t * TP + j], x[j], s0);
      }
      x[t] = (t == li ? 1.f : 0.f) - (s0 + s1);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t)
      if ((t >> 2) == lg) ai[(16 * wave + t) * TP + 16 * wave + li] = x[t];
  }
  __syncthreads();
  // Below the diagonal, one block diagonal at a time: X_ij = -X_ii sum_{k=j}^{i-1} L_ik X_kj,
  // block (wave + dd, wave) on wave `wave`.  The product's output layout is the next
  // product's B operand layout for K = 16 (element m of lane l is row 4 (l / 16) + m).
#pragma unroll
  for (int dd = 1; dd < 4; ++dd) {
    const int j = wave, i = wave + dd;
    if (i < 4) {
      f32x4 p = {0.f, 0.f, 0.f, 0.f};
      for (int kb = j; kb < i; ++kb) {
        float a[4], bb[4];
        lds_run<4>(a, &lm[(16 * i + li) * TP + 16 * kb + 4 * lg]);
#pragma unroll
        for (int m = 0; m < 4; ++m) bb[m] = ai[(16 * kb + 4 * lg + m) * TP + 16 * j + li];
        p = mm_rr<4>(p, a, bb);
      }
      float a[4], bb[4] = {p[0], p[1], p[2], p[3]};
      lds_run<4>(a, &ai[(16 * i + li) * TP + 16 * i + 4 * lg]);
      const f32x4 xr = mm_rr<4>(f32x4{0.f, 0.f, 0.f, 0.f}, a, bb);
#pragma unroll
      for (int v = 0; v < 4; ++v) ai[(16 * i + 4 * lg + v) * TP + 16 * j + li] = -xr[v];
    }
    __syncthreads();
  }
  // Ap = A diag(beta), blocks on and below the diagonal; the shared zero block
  for (int e = tid; e < GC * GC / 4; e += 256) {  // 4 consecutive columns per thread
    const int t = e / (GC / 4), j = (e % (GC / 4)) * 4;
    if ((j >> 4) <= (t >> 4)) {
      const float4 av = *(const float4 *)&ai[t * TP + j], bv = *(const float4 *)&bt[j];
      *(float4 *)&out[WS_AP + t * GC + j] = make_float4(av.x * bv.x, av.y * bv.y, av.z * bv.z, av.w * bv.w);
    }
  }
  if (blockIdx.x == 0 && tid < WS_ZERO) ws[(int64_t)gridDim.x * WS_CHUNK + tid] = 0.f;
}

// (tail o K)^T in LDS: row d, column t, rows of each 32-row band shifted by 16 floats so
// that the four lane groups' stores (rows 32 apart) fall in distinct banks
__device__ __forceinline__ int kt_at(int d, int t) { return d * TP + 16 * (d >> 5) + t; }
constexpr int KT_SIZE = (GDK - 1) * TP + 16 * (GDK / 32 - 1) + GC;

// LDS (floats), only what the four waves share: s [GR][KP] (the rows' state); kt; u, dt
// [GR][TP] (U^T, Dl^T)
constexpr size_t SCAN_LDS = (size_t)(GR * KP + KT_SIZE + 2 * GR * TP) * 4;

// Wave w owns the chunk's steps 16 w .. 16 w + 15 for the products over the chunk's steps,
// and columns 32 w .. 32 w + 31 of the state.  Lane l's A operands (row 16 w + l % 16 of
// K, Q, Ap and M over its lane group's run of columns) come straight from global memory
// into registers, one chunk ahead.
template <bool Y_F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_chunk_scan(
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v, const float *__restrict__ ws,
    const float *st_in, float *st_out, void *__restrict__ y, int T, int Hk, int Hv, int Dv, int nch, int nwg) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *s_s = lds, *kt_s = s_s + GR * KP, *u_s = kt_s + KT_SIZE, *dt_s = u_s + GR * TP;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;  // MFMA operand row / column, lane group
  int nh, r0;
  if (!scan_wg(nwg, Dv / GR, nh, r0)) return;
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int tr = 16 * wave + li;  // this lane's step row of the chunk for its A operands

  // the state rows r0 .. r0 + 15 (element v of lane l of tile h: row 4 (l / 16) + v,
  // column 16 (2 w + h) + l % 16)
  const float *sin = st_in + ((int64_t)nh * Dv + r0) * GDK;
  f32x4 sacc[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) sacc[h][vv] = sin[(4 * lg + vv) * GDK + 16 * (2 * wave + h) + li];
  }
  for (int e = tid; e < GR * GDK; e += 256) s_s[(e / GDK) * KP + e % GDK] = sin[e];

  // one chunk ahead, in registers: the Ap and M runs, V at this lane's output positions,
  // gam, tail (the f32 Q and K rows are read in the chunk, to stay within 256 registers)
  float4 pap[4], pm[4];
  float pv[4], pg, ptl, pgl;
  auto qk_off = [&](int ci) __attribute__((always_inline)) {
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    const int tt = tr < n ? tr : n - 1;  // steps past T re-read the last one (scaled by 0)
    return (((int64_t)b * T + t0 + tt) * Hk + hk) * GDK + 32 * lg;
  };
  // each operand's next-chunk load is issued right after its last use in this chunk, so
  // one set of registers serves both
  auto chunk_ws = [&](int ci) __attribute__((always_inline)) { return ws + ((int64_t)nh * nch + ci) * WS_CHUNK; };
  // lane groups whose block is above the diagonal read the shared zero block instead (no
  // load is conditional: waits for loads are then counted exactly across the chunk loop)
  const bool low = lg <= wave;
  const float *wz = ws + (int64_t)(nwg / (Dv / GR)) * nch * WS_CHUNK;
  auto load_ap = [&](int ci) __attribute__((always_inline)) {
    const float *cw = chunk_ws(ci);
#pragma unroll
    for (int u = 0; u < 4; ++u) pap[u] = ((const float4 *)(low ? &cw[WS_AP + tr * GC + 16 * lg] : wz))[u];
  };
  auto load_m = [&](int ci) __attribute__((always_inline)) {
    const float *cw = chunk_ws(ci);
#pragma unroll
    for (int u = 0; u < 4; ++u) pm[u] = ((const float4 *)(low ? &cw[WS_M + tr * GC + 16 * lg] : wz))[u];
  };
  auto load_q = [&](int ci) __attribute__((always_inline)) {  // Q, V, gam, tail
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    const float *cw = chunk_ws(ci);
    pg = cw[WS_GAM + tr];
    ptl = cw[WS_TAIL + tr];
    pgl = cw[WS_GAM + GC - 1];
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int t = 16 * wave + 4 * lg + vv, tt = t < n ? t : n - 1;
      pv[vv] = ld1f<true>(v, (((int64_t)b * T + t0 + tt) * Hv + hv) * Dv + r0 + li);
    }
  };
  auto k_row = [&](int ci, float *o) __attribute__((always_inline)) {  // this lane's K run
    const int64_t ko = qk_off(ci);
#pragma unroll
    for (int u = 0; u < 4; ++u) ld8f<true>(k, ko + 8 * u, o + 8 * u);
  };

  load_q(0);
  load_ap(0);
  load_m(0);
  // one chunk; FULL chunks (all 64 steps within T) store every y row unconditionally
  auto chunk = [&](int ci, auto full) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full)::value;
    const int t0 = ci * GC, n = FULL ? GC : (T - t0 < GC ? T - t0 : GC);
    const int cn = ci + 1 < nch ? ci + 1 : ci;  // the next chunk (the last reloads itself)
    const bool live = tr < n;
    const float gq = live ? pg : 0.f, tl = live ? ptl : 0.f, gcl = pgl;
    // this chunk's A runs out of the prefetch registers: -gam o K, gam o Q (Ap and M are
    // used where they are)
    float ak[32], aq[32];
    k_row(ci, ak);
#pragma unroll
    for (int m = 0; m < 32; ++m) ak[m] *= -gq;
    {
      const int64_t qo = qk_off(ci);
#pragma unroll
      for (int u = 0; u < 4; ++u) ld8f<true>(q, qo + 8 * u, aq + 8 * u);
    }
#pragma unroll
    for (int m = 0; m < 32; ++m) aq[m] *= gq;
    f32x4 uacc;
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) uacc[vv] = 16 * wave + 4 * lg + vv < n ? pv[vv] : 0.f;
    __syncthreads();  // (A) s_s holds the state before this chunk
    load_q(cn);
    __builtin_amdgcn_sched_barrier(0);  // (issued before the MFMAs, not among them)

    // U = V - (gam o K) S^T and (gam o Q) S^T, over this wave's 16 steps
    float sb[32];
    lds_run<32>(sb, &s_s[li * KP + 32 * lg]);
    uacc = mm_rr<32>(uacc, ak, sb);
    f32x4 yacc = mm_rr<32>(f32x4{0.f, 0.f, 0.f, 0.f}, aq, sb);
    *(f32x4 *)&u_s[li * TP + 16 * wave + 4 * lg] = uacc;  // U^T
    __syncthreads();  // (B) every wave's U rows are in u_s
    {  // (tail o K)^T of this lane's step row; the next chunk's K then goes in flight
      float kr[32];
      k_row(ci, kr);
#pragma unroll
      for (int j = 0; j < 32; ++j) kt_s[kt_at(32 * lg + j, tr)] = tl * kr[j];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Dl = Ap U
    float ub[16];
    lds_run<16>(ub, &u_s[li * TP + 16 * lg]);
    const f32x4 dl = mm_rr<16>(f32x4{0.f, 0.f, 0.f, 0.f}, (const float *)pap, ub);
    __builtin_amdgcn_sched_barrier(0);
    load_ap(cn);
    *(f32x4 *)&dt_s[li * TP + 16 * wave + 4 * lg] = dl;  // Dl^T
    __syncthreads();  // (C) every wave's Dl rows are in dt_s, all of kt_s is written
    // Y = (gam o Q) S^T + M Dl
    float db[16];
    lds_run<16>(db, &dt_s[li * TP + 16 * lg]);
    yacc = mm_rr<16>(yacc, (const float *)pm, db);
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int t = 16 * wave + 4 * lg + vv;
      if (FULL || t < n) {
        const int64_t yi = (((int64_t)b * T + t0 + t) * Hv + hv) * Dv + r0 + li;
        if constexpr (Y_F32)
          ((float *)y)[yi] = yacc[vv];
        else
          ((uint16_t *)y)[yi] = f32_to_bf16_rne(yacc[vv]);
      }
    }
    // S = gam_{C-1} S + Dl^T (tail o K)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int d = 16 * (2 * wave + h) + li;
      float kb[16];
      lds_run<16>(kb, &kt_s[kt_at(d, 16 * lg)]);
      sacc[h] = mm_rr<16>(sacc[h] * gcl, db, kb);
    }
    // every wave read s_s before (B); the next chunk reads it after (A)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) s_s[(4 * lg + vv) * KP + 16 * (2 * wave + h) + li] = sacc[h][vv];
    }
    // M for the next chunk after this chunk's y stores: memory operations complete in
    // order, and a wait for a store (before its data register is reused) then does not
    // also wait for these loads
    __builtin_amdgcn_sched_barrier(0);
    load_m(cn);
  };
  int ci = 0;
  for (; ci < T / GC; ++ci) chunk(ci, std::true_type{});
  if (ci < nch) chunk(ci, std::false_type{});  // the partial last chunk
  float *sout = st_out + ((int64_t)nh * Dv + r0) * GDK;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) sout[(4 * lg + vv) * GDK + 16 * (2 * wave + h) + li] = sacc[h][vv];
  }
}

// x = hi + mid + lo exactly, each part bf16 (the truncation of what is left): x - hi keeps
// at most 16 significant bits and is exact, mid takes the top 8 of them, and the rest (at
// most 8 bits) is exact in bf16.  Returned as bf16 bit patterns.
__device__ __forceinline__ void split3(float x, uint32_t &h, uint32_t &m, uint32_t &l) {
  const uint32_t xb = __float_as_uint(x);
  const float r1 = x - __uint_as_float(xb & 0xFFFF0000u);
  const uint32_t rb = __float_as_uint(r1);
  const float r2 = r1 - __uint_as_float(rb & 0xFFFF0000u);
  h = xb >> 16;
  m = rb >> 16;
  l = __float_as_uint(r2) >> 16;
}

// bf16 LDS layout of the bf16-input scan (in bf16 elements): the state as three split
// planes [GR][SPB]; K^T [GDK][.] with each 32-row band shifted by 32 elements (the four lane
// groups' stores, rows 32 apart, then fall in distinct banks); (tail o Dl)^T as three split
// planes [GR][DPB]
constexpr int SPB = GDK + 8;
constexpr int KTP = GC + 8;
constexpr int DPB = GC + 8;
__device__ __forceinline__ int ktb_at(int d, int t) { return d * KTP + 32 * (d >> 5) + t; }
constexpr int KTB_SIZE = (GDK - 1) * KTP + 32 * (GDK / 32 - 1) + GC;
constexpr size_t SCANB_LDS = (size_t)2 * GR * TP * 4 + (size_t)(3 * GR * SPB + KTB_SIZE + 3 * GR * DPB) * 2;

// The scan for bf16 q, k, v.  Products with K or Q run on the bf16 MFMA, which multiplies
// bf16 values exactly into f32: K S^T and Q S^T with S split into three bf16 planes, and
// the state update Dl^T (tail o K) as (tail o Dl)^T split into three planes times K.  Each
// f32 value is split once, by the lane that holds it.  Dl = Ap U and M Dl (f32 both sides)
// stay on the f32 MFMA.  Layout, chunk loop and prefetch as in gdn_chunk_scan.
template <bool Y_F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_chunk_scan_bf(
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v, const float *__restrict__ ws,
    const float *st_in, float *st_out, void *__restrict__ y, int T, int Hk, int Hv, int Dv, int nch, int nwg) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *u_s = lds, *dt_s = u_s + GR * TP;
  uint16_t *sp = (uint16_t *)(dt_s + GR * TP), *ktb = sp + 3 * GR * SPB, *dp = ktb + KTB_SIZE;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  int nh, r0;
  if (!scan_wg(nwg, Dv / GR, nh, r0)) return;
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int tr = 16 * wave + li;

  // the state rows r0 .. r0 + 15 in accumulators (tile h: row 4 (l / 16) + v, column
  // 16 (2 w + h) + l % 16), and as split planes in LDS
  const float *sin = st_in + ((int64_t)nh * Dv + r0) * GDK;
  f32x4 sacc[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) sacc[h][vv] = sin[(4 * lg + vv) * GDK + 16 * (2 * wave + h) + li];
  }
  auto put_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
        uint32_t p0, p1, p2;
        split3(sacc[h][vv], p0, p1, p2);
        const int o = (4 * lg + vv) * SPB + 16 * (2 * wave + h) + li;
        sp[o] = (uint16_t)p0;
        sp[GR * SPB + o] = (uint16_t)p1;
        sp[2 * GR * SPB + o] = (uint16_t)p2;
      }
    }
  };
  put_state();

  // one chunk ahead, in registers: Q and K row runs (bf16, the A operands as they are), V
  // and gam, tail at this lane's output rows, the Ap and M runs
  bf16x8_t pq[4], pk[4];
  float4 pap[4], pm[4], pg4, ptl4;
  float pv[4], pgl;
  auto qk_off = [&](int ci) __attribute__((always_inline)) {
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    const int tt = tr < n ? tr : n - 1;  // steps past T re-read the last one (scaled by 0)
    return (((int64_t)b * T + t0 + tt) * Hk + hk) * GDK + 32 * lg;
  };
  const bool low = lg <= wave;  // else the lane group's block is above the diagonal: the zero block
  const float *wz = ws + (int64_t)(nwg / (Dv / GR)) * nch * WS_CHUNK;
  auto chunk_ws = [&](int ci) __attribute__((always_inline)) { return ws + ((int64_t)nh * nch + ci) * WS_CHUNK; };
  auto load_ap = [&](int ci) __attribute__((always_inline)) {
    const float *cw = chunk_ws(ci);
#pragma unroll
    for (int u = 0; u < 4; ++u) pap[u] = ((const float4 *)(low ? &cw[WS_AP + tr * GC + 16 * lg] : wz))[u];
  };
  auto load_m = [&](int ci) __attribute__((always_inline)) {
    const float *cw = chunk_ws(ci);
#pragma unroll
    for (int u = 0; u < 4; ++u) pm[u] = ((const float4 *)(low ? &cw[WS_M + tr * GC + 16 * lg] : wz))[u];
  };
  auto load_q = [&](int ci) __attribute__((always_inline)) {  // Q, V, gam, tail
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    const float *cw = chunk_ws(ci);
    pg4 = *(const float4 *)&cw[WS_GAM + 16 * wave + 4 * lg];
    ptl4 = *(const float4 *)&cw[WS_TAIL + 16 * wave + 4 * lg];
    pgl = cw[WS_GAM + GC - 1];
    const bf16x8_t *src = (const bf16x8_t *)((const uint16_t *)q + qk_off(ci));
#pragma unroll
    for (int u = 0; u < 4; ++u) pq[u] = src[u];
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int t = 16 * wave + 4 * lg + vv, tt = t < n ? t : n - 1;
      pv[vv] = bf16_to_f32(((const uint16_t *)v)[(((int64_t)b * T + t0 + tt) * Hv + hv) * Dv + r0 + li]);
    }
  };
  auto load_k = [&](int ci) __attribute__((always_inline)) {
    const bf16x8_t *src = (const bf16x8_t *)((const uint16_t *)k + qk_off(ci));
#pragma unroll
    for (int u = 0; u < 4; ++u) pk[u] = src[u];
  };

  load_q(0);
  load_k(0);
  load_ap(0);
  load_m(0);
  // one chunk; FULL chunks (all 64 steps within T) store every y row unconditionally
  auto chunk = [&](int ci, auto full) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full)::value;
    const int t0 = ci * GC, n = FULL ? GC : (T - t0 < GC ? T - t0 : GC);
    const int cn = ci + 1 < nch ? ci + 1 : ci;  // the next chunk (the last reloads itself)
    // this lane's output rows t = 16 w + 4 (l / 16) + v: gam (0 past T), V, tail
    float gv[4], uv[4];
    const float tlv[4] = {ptl4.x, ptl4.y, ptl4.z, ptl4.w}, gw[4] = {pg4.x, pg4.y, pg4.z, pg4.w};
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const bool live = FULL || 16 * wave + 4 * lg + vv < n;
      gv[vv] = live ? gw[vv] : 0.f;
      uv[vv] = live ? pv[vv] : 0.f;
    }
    const float gcl = pgl;
    bf16x8_t ak[4], aq[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ak[u] = pk[u], aq[u] = pq[u];
    __syncthreads();  // (A) the state planes hold the state before this chunk
    load_q(cn);
    __builtin_amdgcn_sched_barrier(0);

    // K S^T and Q S^T over this wave's 16 steps; U = V - gam o K S^T
    f32x4 ur = {0.f, 0.f, 0.f, 0.f}, yr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int o = li * SPB + 32 * lg + 8 * c;
      const bf16x8_t s0 = *(const bf16x8_t *)&sp[o], s1 = *(const bf16x8_t *)&sp[GR * SPB + o],
                     s2 = *(const bf16x8_t *)&sp[2 * GR * SPB + o];
      ur = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[c], s0, ur, 0, 0, 0);
      yr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq[c], s0, yr, 0, 0, 0);
      ur = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[c], s1, ur, 0, 0, 0);
      yr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq[c], s1, yr, 0, 0, 0);
      ur = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[c], s2, ur, 0, 0, 0);
      yr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq[c], s2, yr, 0, 0, 0);
    }
    f32x4 uacc, yacc;
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      uacc[vv] = __builtin_fmaf(-gv[vv], ur[vv], uv[vv]);
      yacc[vv] = gv[vv] * yr[vv];
    }
    *(f32x4 *)&u_s[li * TP + 16 * wave + 4 * lg] = uacc;  // U^T
    __syncthreads();  // (B) every wave's U rows are in u_s
    // K^T of this lane's step row (bf16 as it is), the elements taken from the vector's
    // 32-bit words (a __bf16 element read out of the vector with __builtin_bit_cast gave
    // element 0 for all eight with this compiler); the next chunk's K then goes in flight
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4_t w = __builtin_bit_cast(u32x4_t, ak[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        ktb[ktb_at(32 * lg + 8 * c + e, tr)] = (uint16_t)(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu);
    }
    load_k(cn);
    __builtin_amdgcn_sched_barrier(0);
    // Dl = Ap U (f32)
    float ub[16];
    lds_run<16>(ub, &u_s[li * TP + 16 * lg]);
    const f32x4 dl = mm_rr<16>(f32x4{0.f, 0.f, 0.f, 0.f}, (const float *)pap, ub);
    __builtin_amdgcn_sched_barrier(0);
    load_ap(cn);
    *(f32x4 *)&dt_s[li * TP + 16 * wave + 4 * lg] = dl;  // Dl^T
    {  // (tail o Dl)^T as split planes: row li, columns 16 w + 4 (l / 16) + v
      uint32_t p0[4], p1[4], p2[4];
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) split3(tlv[vv] * dl[vv], p0[vv], p1[vv], p2[vv]);
      const int o = li * DPB + 16 * wave + 4 * lg;
      *(uint2 *)&dp[o] = make_uint2(p0[0] | (p0[1] << 16), p0[2] | (p0[3] << 16));
      *(uint2 *)&dp[GR * DPB + o] = make_uint2(p1[0] | (p1[1] << 16), p1[2] | (p1[3] << 16));
      *(uint2 *)&dp[2 * GR * DPB + o] = make_uint2(p2[0] | (p2[1] << 16), p2[2] | (p2[3] << 16));
    }
    __syncthreads();  // (C) every wave's Dl rows are in dt_s and dp, all of K^T is written
    // Y = gam o Q S^T + M Dl
    float db[16];
    lds_run<16>(db, &dt_s[li * TP + 16 * lg]);
    yacc = mm_rr<16>(yacc, (const float *)pm, db);
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int t = 16 * wave + 4 * lg + vv;
      if (FULL || t < n) {
        const int64_t yi = (((int64_t)b * T + t0 + t) * Hv + hv) * Dv + r0 + li;
        if constexpr (Y_F32)
          ((float *)y)[yi] = yacc[vv];
        else
          ((uint16_t *)y)[yi] = f32_to_bf16_rne(yacc[vv]);
      }
    }
    // S = gam_{C-1} S + (tail o Dl)^T K
#pragma unroll
    for (int h = 0; h < 2; ++h) sacc[h] *= gcl;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int o = li * DPB + 16 * lg + 8 * c;
      const bf16x8_t a0 = *(const bf16x8_t *)&dp[o], a1 = *(const bf16x8_t *)&dp[GR * DPB + o],
                     a2 = *(const bf16x8_t *)&dp[2 * GR * DPB + o];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bf16x8_t kb = *(const bf16x8_t *)&ktb[ktb_at(16 * (2 * wave + h) + li, 16 * lg + 8 * c)];
        sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, kb, sacc[h], 0, 0, 0);
        sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, kb, sacc[h], 0, 0, 0);
        sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, kb, sacc[h], 0, 0, 0);
      }
    }
    // every wave read the state planes before (B); the next chunk reads them after (A)
    put_state();
    // M for the next chunk after this chunk's y stores (memory operations complete in order)
    __builtin_amdgcn_sched_barrier(0);
    load_m(cn);
  };
  int ci = 0;
  for (; ci < T / GC; ++ci) chunk(ci, std::true_type{});
  if (ci < nch) chunk(ci, std::false_type{});  // the partial last chunk
  float *sout = st_out + ((int64_t)nh * Dv + r0) * GDK;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) sout[(4 * lg + vv) * GDK + 16 * (2 * wave + h) + li] = sacc[h][vv];
  }
}

// prep, then the scan (f32 inputs: gdn_chunk_scan; bf16 inputs: gdn_chunk_scan_bf); both
// scans use under 64 KB of LDS, the default limit
template <bool IN, bool YF>
static hipError_t launch_chunked_t(const GdnArgs &a, float *ws, hipStream_t st) {
  static_assert(SCAN_LDS <= 65536 && SCANB_LDS <= 65536 && PREP_LDS <= 65536, "LDS over the default limit");
  const int nch = (a.T + GC - 1) / GC;
  const int64_t nh = (int64_t)a.B * a.Hv;
  hipLaunchKernelGGL((gdn_chunk_prep<IN>), dim3((unsigned)(nh * nch)), dim3(256), PREP_LDS, st, a.q, a.k, a.g, a.beta,
                     (int)a.beta_f32, ws, a.T, a.Hk, a.Hv, nch);
  const int nwg = (int)(nh * (a.Dv / GR));
  const dim3 grid((unsigned)((nwg + 7) / 8 * 8));
  if constexpr (IN)
    hipLaunchKernelGGL((gdn_chunk_scan<YF>), grid, dim3(256), SCAN_LDS, st, a.q, a.k, a.v, (const float *)ws,
                       a.state_in, a.state_out, a.y, a.T, a.Hk, a.Hv, a.Dv, nch, nwg);
  else
    hipLaunchKernelGGL((gdn_chunk_scan_bf<YF>), grid, dim3(256), SCANB_LDS, st, a.q, a.k, a.v, (const float *)ws,
                       a.state_in, a.state_out, a.y, a.T, a.Hk, a.Hv, a.Dv, nch, nwg);
  return hipGetLastError();
}

}  // namespace

// The shapes the chunked kernels take, at any T >= 1.
static bool gdn_chunked_shape_ok(const GdnArgs &a) {
  if (a.Dk != GDK || a.Dv <= 0 || a.Dv % GR != 0 || a.Hk <= 0 || a.Hv % a.Hk != 0 || a.B <= 0 || a.T <= 0)
    return false;
  const int64_t nch = (a.T + GC - 1) / GC, nh = (int64_t)a.B * a.Hv;
  return nh * nch <= 0x7FFFFFFF && nh * (a.Dv / GR) <= 0x7FFFFFF0;
}

bool gdn_chunked_ok(const GdnArgs &a) { return a.T >= GDN_CHUNKED_MIN_T && gdn_chunked_shape_ok(a); }

size_t gdn_chunked_workspace(const GdnArgs &a) {
  const int64_t nch = (a.T + GC - 1) / GC;
  return ((size_t)a.B * a.Hv * nch * WS_CHUNK + WS_ZERO) * sizeof(float);
}

static hipError_t launch_chunked_any(const GdnArgs &a, float *ws, hipStream_t st) {
  if (a.in_f32) return a.y_f32 ? launch_chunked_t<true, true>(a, ws, st) : launch_chunked_t<true, false>(a, ws, st);
  return a.y_f32 ? launch_chunked_t<false, true>(a, ws, st) : launch_chunked_t<false, false>(a, ws, st);
}

hipError_t launch_gdn_chunked(const GdnArgs &a, void *workspace, hipStream_t st) {
  if (!gdn_chunked_ok(a)) return hipErrorInvalidValue;
  return launch_chunked_any(a, (float *)workspace, st);
}

// ---------------------------------------------------------------- the allocation-free form
//
// The workspace of qmm_gdn_recurrence_noalloc: one array per GPU, held by the process
// until it ends.  Host code reaches it only through the address hipGetSymbolAddress
// returns on each device (the array's name is not a device address on the host).
constexpr size_t GDN_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) float scratch[GDN_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mtx;
void *g_scratch_ptr[MAX_DEVICES] = {};
}  // namespace

size_t gdn_noalloc_scratch_bytes() { return GDN_SCRATCH_BYTES; }

// Largest (b, hv, chunk) count one launch can take in the array.
static int64_t scratch_chunks() { return (int64_t)(GDN_SCRATCH_BYTES / sizeof(float) - WS_ZERO) / WS_CHUNK; }

bool gdn_noalloc_fits(const GdnArgs &a) { return (int64_t)a.Hv <= scratch_chunks(); }

// The array's address on the current device, looked up once per device.
static hipError_t noalloc_scratch(float **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mtx);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = (float *)g_scratch_ptr[dev];
  return hipSuccess;
}

// Arguments of the sub-problem: batches [b0, b0 + nb), steps [t0, t0 + nt).  A sub-problem
// with nt < T has nb = 1, so its rows of q, k, v, g, beta and y are contiguous.
static GdnArgs gdn_part(const GdnArgs &a, int b0, int nb, int t0, int nt) {
  GdnArgs p = a;
  const size_t ie = a.in_f32 ? 4 : 2, be = a.beta_f32 ? 4 : 2, ye = a.y_f32 ? 4 : 2;
  const int64_t step0 = (int64_t)b0 * a.T + t0;  // first (b, t) row of the part
  p.B = nb;
  p.T = nt;
  p.q = (const char *)a.q + step0 * a.Hk * a.Dk * ie;
  p.k = (const char *)a.k + step0 * a.Hk * a.Dk * ie;
  p.v = (const char *)a.v + step0 * a.Hv * a.Dv * ie;
  p.g = a.g + step0 * a.Hv;
  p.beta = (const char *)a.beta + step0 * a.Hv * be;
  p.y = (char *)a.y + step0 * a.Hv * a.Dv * ye;
  const int64_t s0 = (int64_t)b0 * a.Hv * a.Dv * a.Dk;
  p.state_in = a.state_in + s0;
  p.state_out = a.state_out + s0;
  return p;
}

// The recurrence at T >= GDN_CHUNKED_MIN_T with the workspace in the array.  A call whose
// workspace exceeds the array runs as several launches on the same stream: groups of whole
// batches, or for one batch, runs of whole 64-step chunks, the state carried through
// state_out.  Every (b, hv, chunk) is computed by the same instructions as in one launch,
// so the results are identical bit for bit.  Needs gdn_noalloc_fits(a).
hipError_t launch_gdn_chunked_noalloc(const GdnArgs &a, hipStream_t st) {
  if (!gdn_chunked_ok(a) || !gdn_noalloc_fits(a)) return hipErrorInvalidValue;
  float *ws = nullptr;
  hipError_t e = noalloc_scratch(&ws);
  if (e != hipSuccess) return e;
  const int64_t cap = scratch_chunks(), nch = (a.T + GC - 1) / GC, per_batch = (int64_t)a.Hv * nch;
  if ((int64_t)a.B * per_batch <= cap) return launch_chunked_any(a, ws, st);
  if (per_batch <= cap) {  // groups of whole batches
    const int group = (int)(cap / per_batch);
    for (int b0 = 0; b0 < a.B && e == hipSuccess; b0 += group)
      e = launch_chunked_any(gdn_part(a, b0, a.B - b0 < group ? a.B - b0 : group, 0, a.T), ws, st);
    return e;
  }
  const int seg = (int)(cap / a.Hv) * GC;  // steps per launch, whole chunks
  for (int b = 0; b < a.B && e == hipSuccess; ++b)
    for (int t0 = 0; t0 < a.T && e == hipSuccess; t0 += seg) {
      GdnArgs p = gdn_part(a, b, 1, t0, a.T - t0 < seg ? a.T - t0 : seg);
      if (t0 > 0) p.state_in = p.state_out;  // the state the previous run left
      e = launch_chunked_any(p, ws, st);
    }
  return e;
}

}  // namespace qmm
