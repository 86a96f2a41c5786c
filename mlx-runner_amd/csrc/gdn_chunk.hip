// Chunked (matrix) form of the gated-delta recurrence for long T (prefill), on
// the f32 MFMA.  Same results as the step-by-step kernel in gdn.hip (to f32
// rounding): for each (b, value head hv, key head hk = hv / (Hv / Hk)) and
// chunk of C steps t = 0..C-1 with S0 the state before the chunk,
//   G_t = sum_{i <= t} log g_i (f64),  D_tj = exp(G_t - G_j) for j <= t,
//   gam_t = exp(G_t),  tail_t = exp(G_{C-1} - G_t),
//   A   = (I + tril(diag(beta) (D o K K^T), -1))^-1,  Ap = A diag(beta),
//   W   = Ap (gam o K) (stored negated),  M = tril(D o Q K^T)  (diagonal included),
//   Dl  = Ap V - W S0^T                          [C, Dv]  (the chunk's deltas)
//   Y   = (gam o Q) S0^T + M Dl                  [C, Dv]
//   S1  = gam_{C-1} S0 + Dl^T (tail o K)         [Dv, Dk]
// which unrolls S_t = g_t S_{t-1} + dlt_t k_t^T, dlt_t = beta_t (v_t - g_t S_{t-1} k_t),
// y_t = S_t q_t over the chunk.  Steps past T are padded with g = 1, beta = 0
// and zero q, k, v: they leave the state as it is and write nothing.
//
// gdn_chunk_prep, one workgroup per (b, hv, chunk): K K^T, Q K^T and W on the
// MFMA, the triangular inverse by forward substitution (one column per lane),
// and Ap, W, M, gam, tail into a workspace.
// gdn_chunk_scan, one workgroup per (b, hv, 16 state rows): the chunks in
// order; the rows' state stays in MFMA accumulators (wave w holds columns
// 32 w .. 32 w + 31), and per chunk the five products above run as 16x16 MFMA
// tiles from operands staged in LDS.
#include <type_traits>

#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

constexpr int GC = 64;    // steps per chunk
constexpr int GDK = 128;  // key head dim
constexpr int GR = 16;    // state rows per scan workgroup
constexpr int KP = GDK + 4;  // LDS row pitch of [.][GDK] arrays (floats)
constexpr int CP = GC + 1;   // LDS row pitch of [.][GC] arrays
constexpr int RP = GR + 1;   // LDS row pitch of [.][GR] arrays

// workspace per (b, hv, chunk), in floats
constexpr int WS_W = 0;
constexpr int WS_AP = WS_W + GC * GDK;
constexpr int WS_M = WS_AP + GC * GC;
constexpr int WS_GAM = WS_M + GC * GC;
constexpr int WS_TAIL = WS_GAM + GC;
constexpr int WS_CHUNK = WS_TAIL + GC;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// D += A B for one 16 x 16 tile: A(i, k) and B(k, j) from the accessors, K a multiple
// of 4.  v_mfma_f32_16x16x4f32: lane l supplies A(l % 16, k0 + l / 16) and
// B(k0 + l / 16, l % 16); output element v of lane l is D(4 (l / 16) + v, l % 16).
template <typename FA, typename FB>
__device__ __forceinline__ f32x4 mm_tile(f32x4 c, int K, int lane, FA a_of, FB b_of) {
  const int i = lane & 15, kk = lane >> 4;
  for (int k0 = 0; k0 < K; k0 += 4) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a_of(i, k0 + kk), b_of(k0 + kk, i), c, 0, 0, 0);
  return c;
}

template <bool F32>
__device__ __forceinline__ void ld8f(const void *p, int64_t i, float (&o)[8]) {
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


// q and k rows t0 .. t0 + n - 1 of key head hk into [GC][KP] LDS arrays as f32 (zero past n):
// every load is issued before the first store
template <bool IN_F32>
__device__ __forceinline__ void stage_qk(float *qd, float *kd, const void *q, const void *k, int b, int t0, int n,
                                         int T, int Hk, int hk, int tid) {
  constexpr int PER = GC * GDK / 8 / 256;  // 8-element pieces per thread per array
  float rq[PER][8], rk[PER][8];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = tid + 256 * u, t = e / (GDK / 8), d = (e % (GDK / 8)) * 8;
    const int tt = t < n ? t : n - 1;  // rows past n re-read row n - 1 (zeroed below)
    const int64_t off = (((int64_t)b * T + t0 + tt) * Hk + hk) * GDK + d;
    ld8f<IN_F32>(q, off, rq[u]);
    ld8f<IN_F32>(k, off, rk[u]);
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = tid + 256 * u, t = e / (GDK / 8), d = (e % (GDK / 8)) * 8;
    const bool live = t < n;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qd[t * KP + d + j] = live ? rq[u][j] : 0.f;
      kd[t * KP + d + j] = live ? rk[u][j] : 0.f;
    }
  }
}

constexpr int LP = GC + 4;  // LDS row pitch of the L matrix (16-byte aligned rows for vector reads)

// LDS (floats): ks, qs [GC][KP]; lm [GC][LP]; mm, ai [GC][CP]; gd (doubles) [GC]; bt, gam [GC]
constexpr size_t PREP_LDS = (size_t)(2 * GC * KP + GC * LP + 2 * GC * CP + 2 * GC) * 4 + GC * 8;

template <bool IN_F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gdn_chunk_prep(const void *__restrict__ q, const void *__restrict__ k,
                                                      const float *__restrict__ g, const void *__restrict__ beta,
                                                      int beta_f32, float *__restrict__ ws, int T, int Hk, int Hv,
                                                      int nch) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *ks = lds, *qs = ks + GC * KP, *lm = qs + GC * KP, *mm = lm + GC * LP, *ai = mm + GC * CP;
  float *bt = ai + GC * CP, *gam = bt + GC;
  double *gd = (double *)(gam + GC);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ci = blockIdx.x % nch, nh = blockIdx.x / nch;  // nh = b * Hv + hv
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
  float *out = ws + ((int64_t)nh * nch + ci) * WS_CHUNK;

  if (tid < GC) {
    double a = 0.0;
    float be = 0.f;
    if (tid < n) {
      const int64_t gi = ((int64_t)b * T + t0 + tid) * Hv + hv;
      const double gv = (double)g[gi];
      a = gv > 0.0 ? log(gv) : -1.0e4;  // g = 0 wipes the state: exp of the difference underflows to 0
      be = beta_f32 ? ((const float *)beta)[gi] : bf16_to_f32(((const uint16_t *)beta)[gi]);
    }
    gd[tid] = a;
    bt[tid] = be;
  }
  stage_qk<IN_F32>(qs, ks, q, k, b, t0, n, T, Hk, hk, tid);
  __syncthreads();
  if (tid == 0) {  // inclusive prefix sum of the log-decays, in f64
    double s = 0.0;
    for (int t = 0; t < GC; ++t) {
      s += gd[t];
      gd[t] = s;
    }
  }
  __syncthreads();
  if (tid < GC) {
    gam[tid] = (float)exp(gd[tid]);
    out[WS_GAM + tid] = gam[tid];
    out[WS_TAIL + tid] = (float)exp(gd[GC - 1] - gd[tid]);
  }

  // K K^T and Q K^T, row block tb = wave, column blocks jb <= tb (the rest is zero)
  {
    const int tb = wave;
    for (int jb = 0; jb < 4; ++jb) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
      if (jb <= tb) {
        kk = mm_tile(kk, GDK, lane, [&](int i, int c) { return ks[(16 * tb + i) * KP + c]; },
                     [&](int c, int j) { return ks[(16 * jb + j) * KP + c]; });
        qk = mm_tile(qk, GDK, lane, [&](int i, int c) { return qs[(16 * tb + i) * KP + c]; },
                     [&](int c, int j) { return ks[(16 * jb + j) * KP + c]; });
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 16 * tb + 4 * (lane >> 4) + v, j = 16 * jb + (lane & 15);
        const float d = j <= t ? (float)exp(gd[t] - gd[j]) : 0.f;
        lm[t * LP + j] = j < t ? bt[t] * d * kk[v] : 0.f;
        mm[t * CP + j] = d * qk[v];
      }
    }
  }
  __syncthreads();

  // A = (I + L)^-1 by forward substitution, column c per lane of wave 0, the column in
  // registers: col[t] = delta_tc - sum_{j<t} L[t][j] col[j].  Rows above c come out zero by
  // themselves (every earlier entry of the column is zero), so all lanes run the same code;
  // L's rows are broadcast reads, and each sum runs in four partial sums.
  if (wave == 0) {
    const int c = lane;
    float col[GC];
#pragma unroll
    for (int t = 0; t < GC; ++t) {
      float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j0 = 0; j0 < (t & ~3); j0 += 4) {
        const float4 l4 = *(const float4 *)&lm[t * LP + j0];
        a[0] = __builtin_fmaf(l4.x, col[j0], a[0]);
        a[1] = __builtin_fmaf(l4.y, col[j0 + 1], a[1]);
        a[2] = __builtin_fmaf(l4.z, col[j0 + 2], a[2]);
        a[3] = __builtin_fmaf(l4.w, col[j0 + 3], a[3]);
      }
#pragma unroll
      for (int j = t & ~3; j < t; ++j) a[j & 3] = __builtin_fmaf(lm[t * LP + j], col[j], a[j & 3]);
      col[t] = (t == c ? 1.f : 0.f) - ((a[0] + a[1]) + (a[2] + a[3]));
    }
#pragma unroll
    for (int t = 0; t < GC; ++t) ai[t * CP + c] = col[t];
  }
  __syncthreads();
  for (int e = tid; e < GC * GC; e += 256) {  // Ap = A diag(beta), M
    const int t = e / GC, j = e % GC;
    const float ap = ai[t * CP + j] * bt[j];
    ai[t * CP + j] = ap;
    out[WS_AP + e] = ap;
    out[WS_M + e] = mm[t * CP + j];
  }
  __syncthreads();
  // W = Ap (gam o K): row block tb = wave, column blocks db = 0..7
  {
    const int tb = wave;
    for (int db = 0; db < GDK / 16; ++db) {
      f32x4 w = {0.f, 0.f, 0.f, 0.f};
      w = mm_tile(w, GC, lane, [&](int i, int c) { return ai[(16 * tb + i) * CP + c]; },
                  [&](int c, int j) { return gam[c] * ks[c * KP + 16 * db + j]; });
#pragma unroll
      for (int v = 0; v < 4; ++v) out[WS_W + (16 * tb + 4 * (lane >> 4) + v) * GDK + 16 * db + (lane & 15)] = -w[v];
    }
  }
}

// D += A B for one 16 x 16 tile over K = 4 NK, lane group g = l / 16 taking k = NK g + m
// (m < NK): the order of the terms of a sum is free, and a lane's operands are then NK
// consecutive floats of a row of A (from arow) and of a column of B (from bcol, B stored
// transposed), read with float4 loads before the MFMAs run back to back.
template <int NK>
__device__ __forceinline__ f32x4 mm_run(f32x4 c, const float *arow, const float *bcol) {
  float a[NK], b[NK];
#pragma unroll
  for (int m = 0; m < NK; m += 4) {
    *(float4 *)&a[m] = *(const float4 *)(arow + m);
    *(float4 *)&b[m] = *(const float4 *)(bcol + m);
  }
#pragma unroll
  for (int m = 0; m < NK; ++m) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m], b[m], c, 0, 0, 0);
  return c;
}

constexpr int TP = GC + 4;  // LDS row pitch of [.][GC] arrays read as float4 runs

// As mm_run, with this lane's A run already in registers.
template <int NK>
__device__ __forceinline__ f32x4 mm_reg(f32x4 c, const float (&a)[NK], const float *bcol) {
  float b[NK];
#pragma unroll
  for (int m = 0; m < NK; m += 4) *(float4 *)&b[m] = *(const float4 *)(bcol + m);
#pragma unroll
  for (int m = 0; m < NK; ++m) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m], b[m], c, 0, 0, 0);
  return c;
}

// LDS (floats), only what the four waves share: kt [GDK][TP] ((tail o K)^T); s [GR][KP]
// (the rows' state); vt, dt [GR][TP] (V^T, Dl^T)
constexpr size_t SCAN_LDS = (size_t)(GDK * TP + GR * KP + 2 * GR * TP) * 4;

// Wave w owns the chunk's steps 16 w .. 16 w + 15 for the products over the chunk's steps,
// and columns 32 w .. 32 w + 31 of the state.  Lane l's A operands (rows 16 w + l % 16 of
// -W, gam o Q, Ap and M, over the lane group's run of columns) come straight from global
// memory into registers, one chunk ahead.
template <bool IN_F32, bool Y_F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_chunk_scan(
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v, const float *__restrict__ ws,
    const float *st_in, float *st_out, void *__restrict__ y, int T, int Hk, int Hv, int Dv, int nch) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float *kt_s = lds, *s_s = kt_s + GDK * TP, *vt_s = s_s + GR * KP, *dt_s = vt_s + GR * TP;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;  // MFMA operand row / column, lane group
  // workgroup id = head + heads * row group: the row groups of a head, which read the same
  // chunk operands, are a multiple of the head count apart, so with a multiple of 8 heads
  // they land on one XCD (workgroups are dealt to the 8 XCDs in turn) and share its L2
  const int nheads = gridDim.x / (Dv / GR);
  const int nh = blockIdx.x % nheads, r0 = (blockIdx.x / nheads) * GR;
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

  // one chunk ahead, in registers: the A runs, and this thread's share of K (t-major:
  // thread i takes step i % 64, columns 8 (i / 64) + 32 u) and of V
  constexpr int NKP = GC * GDK / 8 / 256;  // 8-element K pieces per thread
  float4 pw[8], pap[4], pm[4];
  uint4 pq[4];  // 32 bf16 (f32 inputs: read in the chunk, not ahead, to stay within 256 registers)
  float pg, pgl;  // gam of this lane's step row; gam_{C-1}
  float pk[NKP][8], ptl, pv[4];
  const int kt_t = tid & 63, kt_d = (tid >> 6) * 8;
  const int vt = tid >> 2, vr = (tid & 3) * 4;
  auto load_chunk = [&](int ci) __attribute__((always_inline)) {
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    const float *cw = ws + ((int64_t)nh * nch + ci) * WS_CHUNK;
#pragma unroll
    for (int u = 0; u < 8; ++u) pw[u] = *(const float4 *)&cw[WS_W + tr * GDK + 32 * lg + 4 * u];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pap[u] = *(const float4 *)&cw[WS_AP + tr * GC + 16 * lg + 4 * u];
      pm[u] = *(const float4 *)&cw[WS_M + tr * GC + 16 * lg + 4 * u];
    }
    pg = cw[WS_GAM + tr];
    pgl = cw[WS_GAM + GC - 1];
    ptl = cw[WS_TAIL + kt_t];
    {
      const int tq = tr < n ? tr : n - 1;  // steps past T re-read the last one (their gam is used as 0)
      const int64_t qo = (((int64_t)b * T + t0 + tq) * Hk + hk) * GDK + 32 * lg;
      if constexpr (!IN_F32) {
#pragma unroll
        for (int u = 0; u < 4; ++u) pq[u] = ((const uint4 *)((const uint16_t *)q + qo))[u];
      }
    }
    {
      const int tk = kt_t < n ? kt_t : n - 1;
#pragma unroll
      for (int u = 0; u < NKP; ++u)
        ld8f<IN_F32>(k, (((int64_t)b * T + t0 + tk) * Hk + hk) * GDK + kt_d + 32 * u, pk[u]);
    }
    {
      const int tt = vt < n ? vt : n - 1;
      const int64_t vo = (((int64_t)b * T + t0 + tt) * Hv + hv) * Dv + r0 + vr;
#pragma unroll
      for (int j = 0; j < 4; ++j) pv[j] = ld1f<IN_F32>(v, vo + j);
    }
  };

  load_chunk(0);
  for (int ci = 0; ci < nch; ++ci) {
    const int t0 = ci * GC, n = T - t0 < GC ? T - t0 : GC;
    // this chunk's A runs out of the prefetch registers; K^T and V^T into LDS
    float aw[GDK / 4], aq[GDK / 4], aap[GC / 4], am[GC / 4];
#pragma unroll
    for (int u = 0; u < 8; ++u) *(float4 *)&aw[4 * u] = pw[u];
#pragma unroll
    for (int u = 0; u < 4; ++u) *(float4 *)&aap[4 * u] = pap[u], *(float4 *)&am[4 * u] = pm[u];
    const float gq = tr < n ? pg : 0.f;
    if constexpr (IN_F32) {
      const int tq = tr < n ? tr : n - 1;
      const float *qp = (const float *)q + (((int64_t)b * T + t0 + tq) * Hk + hk) * GDK + 32 * lg;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 f = ((const float4 *)qp)[u];
        aq[4 * u] = gq * f.x, aq[4 * u + 1] = gq * f.y, aq[4 * u + 2] = gq * f.z, aq[4 * u + 3] = gq * f.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t wv[4] = {pq[u].x, pq[u].y, pq[u].z, pq[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          aq[8 * u + 2 * j] = gq * __uint_as_float(wv[j] << 16);
          aq[8 * u + 2 * j + 1] = gq * __uint_as_float(wv[j] & 0xFFFF0000u);
        }
      }
    }
    const float gcl = pgl;
    {
      const float tl = kt_t < n ? ptl : 0.f;
#pragma unroll
      for (int u = 0; u < NKP; ++u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) kt_s[(kt_d + 32 * u + j) * TP + kt_t] = tl * pk[u][j];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) vt_s[(vr + j) * TP + vt] = vt < n ? pv[j] : 0.f;
    __syncthreads();
    load_chunk(ci + 1 < nch ? ci + 1 : ci);  // the next chunk in flight (the last reloads itself)
    __builtin_amdgcn_sched_barrier(0);       // (issued before the MFMAs, not among them)

    // Dl = Ap V - W S^T, stored transposed
    f32x4 dl = {0.f, 0.f, 0.f, 0.f};
    dl = mm_reg<GC / 4>(dl, aap, &vt_s[li * TP + (GC / 4) * lg]);
    dl = mm_reg<GDK / 4>(dl, aw, &s_s[li * KP + (GDK / 4) * lg]);
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) dt_s[li * TP + 16 * wave + 4 * lg + vv] = dl[vv];
    // Y = (gam o Q) S^T + M Dl
    f32x4 yv = {0.f, 0.f, 0.f, 0.f};
    yv = mm_reg<GDK / 4>(yv, aq, &s_s[li * KP + (GDK / 4) * lg]);
    __syncthreads();  // every wave's Dl rows are in dt_s
    yv = mm_reg<GC / 4>(yv, am, &dt_s[li * TP + (GC / 4) * lg]);
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int t = 16 * wave + 4 * lg + vv;
      if (t < n) {
        const int64_t yi = (((int64_t)b * T + t0 + t) * Hv + hv) * Dv + r0 + li;
        if constexpr (Y_F32)
          ((float *)y)[yi] = yv[vv];
        else
          ((uint16_t *)y)[yi] = f32_to_bf16_rne(yv[vv]);
      }
    }
    // S = gam_{C-1} S + Dl^T (tail o K)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int db = 2 * wave + h;
      sacc[h] = mm_run<GC / 4>(sacc[h] * gcl, &dt_s[li * TP + (GC / 4) * lg],
                               &kt_s[(16 * db + li) * TP + (GC / 4) * lg]);
    }
    __syncthreads();  // every wave is done reading s_s, dt_s, kt_s and vt_s
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) s_s[(4 * lg + vv) * KP + 16 * (2 * wave + h) + li] = sacc[h][vv];
    }
    // (the next chunk's staging ends with a barrier before s_s is read)
  }
  float *sout = st_out + ((int64_t)nh * Dv + r0) * GDK;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) sout[(4 * lg + vv) * GDK + 16 * (2 * wave + h) + li] = sacc[h][vv];
  }
}

template <bool IN, bool YF>
static hipError_t launch_chunked_t(const GdnArgs &a, float *ws, hipStream_t st) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)gdn_chunk_prep<IN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)PREP_LDS);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void *)gdn_chunk_scan<IN, YF>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)SCAN_LDS);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int nch = (a.T + GC - 1) / GC;
  const int64_t nh = (int64_t)a.B * a.Hv;
  hipLaunchKernelGGL((gdn_chunk_prep<IN>), dim3((unsigned)(nh * nch)), dim3(256), PREP_LDS, st, a.q, a.k, a.g, a.beta,
                     (int)a.beta_f32, ws, a.T, a.Hk, a.Hv, nch);
  hipLaunchKernelGGL((gdn_chunk_scan<IN, YF>), dim3((unsigned)(nh * (a.Dv / GR))), dim3(256), SCAN_LDS, st, a.q, a.k,
                     a.v, (const float *)ws, a.state_in, a.state_out, a.y, a.T, a.Hk, a.Hv, a.Dv, nch);
  return hipGetLastError();
}

}  // namespace

bool gdn_chunked_ok(const GdnArgs &a) {
  if (a.Dk != GDK || a.Dv <= 0 || a.Dv % GR != 0 || a.Hk <= 0 || a.Hv % a.Hk != 0 || a.B <= 0) return false;
  if (a.T < GDN_CHUNKED_MIN_T) return false;
  const int64_t nch = (a.T + GC - 1) / GC, nh = (int64_t)a.B * a.Hv;
  return nh * nch <= 0x7FFFFFFF && nh * (a.Dv / GR) <= 0x7FFFFFFF;
}

size_t gdn_chunked_workspace(const GdnArgs &a) {
  const int64_t nch = (a.T + GC - 1) / GC;
  return (size_t)a.B * a.Hv * nch * WS_CHUNK * sizeof(float);
}

hipError_t launch_gdn_chunked(const GdnArgs &a, void *workspace, hipStream_t st) {
  if (!gdn_chunked_ok(a)) return hipErrorInvalidValue;
  float *ws = (float *)workspace;
  if (a.in_f32) return a.y_f32 ? launch_chunked_t<true, true>(a, ws, st) : launch_chunked_t<true, false>(a, ws, st);
  return a.y_f32 ? launch_chunked_t<false, true>(a, ws, st) : launch_chunked_t<false, false>(a, ws, st);
}

}  // namespace qmm
