// Packed gated-delta (GDN) recurrence on gfx950: the kernel mlx-runner launches
// through gdnKernelRun (src/model.zig:284-319; the Metal source is
// src/gdn_packed.metal), which gdnForward uses when fusedEligible holds
// (src/model.zig:322-329, :1158).  For each batch b, value head hv (key head
// hk = hv / (Hv / Hk)) and state row r of S[Dv, Dk] (f32), per step t:
//
//   S[r, :] *= g[t];  kv = S[r, :] . k[t];  dlt = (v[t, r] - kv) * beta[t]
//   S[r, :] += dlt * k[t];  y[t, r] = S[r, :] . q[t]
//
// Mapping: a workgroup of 4 waves owns 16 rows of one (b, hv); 16 lanes hold
// one row, 8 state values each (Dk = 128), in registers for all T steps.  The
// two dot products per step reduce over the row's 16 lanes with 4 DPP adds.
// The per-step inputs shared by the workgroup's rows (q and k of head hk, g,
// beta, and v of its 16 rows) are staged into LDS 16 steps at a time, converted
// to f32 once, with the next block's loads in flight while the current block
// is computed; y goes out 16 steps at a time as coalesced rows.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

constexpr int GDN_DK = 128;  // key head dim served (the reference's packed path requires 128)
constexpr int GDN_TB = 16;   // steps staged per block

// Sum over the 16 lanes of a row; every lane of the row receives the same value
// (each step adds a lane's value to its partner's, a commutative pair).
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
  return v;
}

template <bool F32>
__device__ __forceinline__ float ld_elem(const void *p, int64_t i) {
  if constexpr (F32)
    return ((const float *)p)[i];
  else
    return bf16_to_f32(((const uint16_t *)p)[i]);
}

// 8 consecutive elements starting at element i (16-byte aligned for bf16, 32-byte for f32).
template <bool F32>
__device__ __forceinline__ void ld8(const void *p, int64_t i, float (&o)[8]) {
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

// Workgroup barrier for LDS data only (no wait on global memory).
__device__ __forceinline__ void gdn_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// IN_F32: q, k, v are float32 (else bfloat16).  Y_F32: y is float32 (else bfloat16, RNE).
// beta is float32 or bfloat16 (beta_f32); g and the state are float32.  ONE: T fits one
// staged block (decode), so no next block is loaded: the reload the loop issues after its
// last block would cost the call a memory round trip (a separate instance, so that the
// long-T loop keeps its code).
template <bool IN_F32, bool Y_F32, bool ONE>
__global__ __launch_bounds__(256) void gdn_kernel(const void *__restrict__ q, const void *__restrict__ k,
                                                  const void *__restrict__ v, const float *__restrict__ g,
                                                  const void *__restrict__ beta, int beta_f32,
                                                  const float *st_in, float *st_out,
                                                  void *__restrict__ y, int T, int Hk, int Hv, int Dv) {
  __shared__ __attribute__((aligned(16))) float qs[2][GDN_TB][GDN_DK];
  __shared__ __attribute__((aligned(16))) float ks[2][GDN_TB][GDN_DK];
  __shared__ float vs[2][GDN_TB][16];
  __shared__ float gs[2][GDN_TB], bs[2][GDN_TB];
  __shared__ float ys[GDN_TB][16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int groups = (Dv + 15) >> 4;
  const int nh = blockIdx.x / groups, grp = blockIdx.x - nh * groups;  // nh = b * Hv + hv
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int r16 = wave * 4 + (lane >> 4);  // this lane's row within the group
  const int row = grp * 16 + r16;
  const bool live = row < Dv;
  const int seg = (lane & 15) * 8;  // this lane's 8 state columns

  // staging share of thread tid for a block starting at step t0: q and k elements
  // [8 (tid % 16), +8) of step tid / 16; v of row tid % 16 at step tid / 16; g, beta of step tid
  const int st = tid >> 4, d0 = (tid & 15) * 8;
  float rq[8], rk[8], rv = 0.f, rg = 0.f, rb = 0.f;
  auto stage_load = [&](int t0) __attribute__((always_inline)) {
    int t = t0 + st;
    t = t < T ? t : T - 1;  // steps past T read step T-1 (never used)
    const int64_t qk = (((int64_t)b * T + t) * Hk + hk) * GDN_DK + d0;
    ld8<IN_F32>(q, qk, rq);
    ld8<IN_F32>(k, qk, rk);
    const int vr = grp * 16 + (tid & 15);
    rv = ld_elem<IN_F32>(v, (((int64_t)b * T + t) * Hv + hv) * Dv + (vr < Dv ? vr : Dv - 1));
    if (tid < GDN_TB) {
      int tg = t0 + tid;
      tg = tg < T ? tg : T - 1;
      const int64_t gi = ((int64_t)b * T + tg) * Hv + hv;
      rg = g[gi];
      rb = beta_f32 ? ((const float *)beta)[gi] : bf16_to_f32(((const uint16_t *)beta)[gi]);
    }
  };
  auto stage_store = [&](int buf) __attribute__((always_inline)) {
    *(float4 *)&qs[buf][st][d0] = make_float4(rq[0], rq[1], rq[2], rq[3]);
    *(float4 *)&qs[buf][st][d0 + 4] = make_float4(rq[4], rq[5], rq[6], rq[7]);
    *(float4 *)&ks[buf][st][d0] = make_float4(rk[0], rk[1], rk[2], rk[3]);
    *(float4 *)&ks[buf][st][d0 + 4] = make_float4(rk[4], rk[5], rk[6], rk[7]);
    vs[buf][st][tid & 15] = rv;
    if (tid < GDN_TB) {
      gs[buf][tid] = rg;
      bs[buf][tid] = rb;
    }
  };

  // the state row segment, in registers for all steps
  float s[8];
  const int64_t so = ((int64_t)nh * Dv + (live ? row : 0)) * GDN_DK + seg;
  {
    const float4 a = *(const float4 *)(st_in + so), c = *(const float4 *)(st_in + so + 4);
    s[0] = a.x, s[1] = a.y, s[2] = a.z, s[3] = a.w, s[4] = c.x, s[5] = c.y, s[6] = c.z, s[7] = c.w;
  }

  stage_load(0);
  stage_store(0);
  gdn_lds_barrier();
  const int nblk = ONE ? 1 : (T + GDN_TB - 1) / GDN_TB;
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1, t0 = blk * GDN_TB;
    if constexpr (!ONE) stage_load(t0 + GDN_TB < T ? t0 + GDN_TB : t0);  // next block in flight (the last block reloads itself)
    const int steps = T - t0 < GDN_TB ? T - t0 : GDN_TB;
    for (int i = 0; i < steps; ++i) {
      float qv[8], kv8[8];
      *(float4 *)&qv[0] = *(const float4 *)&qs[buf][i][seg];
      *(float4 *)&qv[4] = *(const float4 *)&qs[buf][i][seg + 4];
      *(float4 *)&kv8[0] = *(const float4 *)&ks[buf][i][seg];
      *(float4 *)&kv8[4] = *(const float4 *)&ks[buf][i][seg + 4];
      const float gt = gs[buf][i], bt = bs[buf][i], vt = vs[buf][i][r16];
      float kv = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[e] *= gt;
        kv = __builtin_fmaf(s[e], kv8[e], kv);
      }
      kv = row16_sum(kv);
      const float dlt = (vt - kv) * bt;
      float o = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[e] = __builtin_fmaf(kv8[e], dlt, s[e]);
        o = __builtin_fmaf(s[e], qv[e], o);
      }
      o = row16_sum(o);
      if ((lane & 15) == 0) ys[i][r16] = o;
    }
    gdn_lds_barrier();  // ys complete; every wave is done reading this block's stage
    if (tid < steps * 16) {
      const int t = t0 + (tid >> 4), r = grp * 16 + (tid & 15);
      const int64_t yi = (((int64_t)b * T + t) * Hv + hv) * Dv + r;
      const float yvv = ys[tid >> 4][tid & 15];
      if (r < Dv) {
        if constexpr (Y_F32)
          ((float *)y)[yi] = yvv;
        else
          ((uint16_t *)y)[yi] = f32_to_bf16_rne(yvv);
      }
    }
    if constexpr (!ONE) {
      stage_store(buf ^ 1);
      gdn_lds_barrier();
    }
  }
  if (live) {
    *(float4 *)(st_out + so) = make_float4(s[0], s[1], s[2], s[3]);
    *(float4 *)(st_out + so + 4) = make_float4(s[4], s[5], s[6], s[7]);
  }
}

// T <= GDN_SHORT (a decode step, or the few steps of a speculative verify): the same mapping
// and arithmetic as gdn_kernel (the results are equal bit for bit), without the staging: each
// lane loads its own 8 elements of q and k, its row's v and the head's g and beta for every
// step straight from global memory, all before the first step, together with its state, and
// the lane that ends a row's reduction stores y.  No LDS and no barrier.
constexpr int GDN_SHORT = 4;

template <bool IN_F32, bool Y_F32>
__global__ __launch_bounds__(256) void gdn_short_kernel(int T, int Hk, int Hv, int Dv, int beta_f32,
                                                        const float *st_in, const void *__restrict__ q,
                                                        const void *__restrict__ k, const void *__restrict__ v,
                                                        const float *__restrict__ g, const void *__restrict__ beta,
                                                        float *st_out, void *__restrict__ y) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int groups = (Dv + 15) >> 4;
  const int nh = blockIdx.x / groups, grp = blockIdx.x - nh * groups;  // nh = b * Hv + hv
  const int b = nh / Hv, hv = nh - b * Hv, hk = hv / (Hv / Hk);
  const int r16 = wave * 4 + (lane >> 4);
  const int row = grp * 16 + r16;
  const bool live = row < Dv;
  const int seg = (lane & 15) * 8;
  const int rr = live ? row : 0;

  float s[8];
  const int64_t so = ((int64_t)nh * Dv + rr) * GDN_DK + seg;
  {
    const float4 a = *(const float4 *)(st_in + so), c = *(const float4 *)(st_in + so + 4);
    s[0] = a.x, s[1] = a.y, s[2] = a.z, s[3] = a.w, s[4] = c.x, s[5] = c.y, s[6] = c.z, s[7] = c.w;
  }
  float qv[GDN_SHORT][8], kv8[GDN_SHORT][8], vt[GDN_SHORT], gt[GDN_SHORT], bt[GDN_SHORT];
#pragma unroll
  for (int t = 0; t < GDN_SHORT; ++t) {
    if (t < T) {
      const int64_t bt_ = (int64_t)b * T + t;  // (batch, step)
      const int64_t qk = (bt_ * Hk + hk) * GDN_DK + seg;
      ld8<IN_F32>(q, qk, qv[t]);
      ld8<IN_F32>(k, qk, kv8[t]);
      vt[t] = ld_elem<IN_F32>(v, (bt_ * Hv + hv) * Dv + rr);
      const int64_t gi = bt_ * Hv + hv;
      gt[t] = g[gi];
      bt[t] = beta_f32 ? ((const float *)beta)[gi] : bf16_to_f32(((const uint16_t *)beta)[gi]);
    }
  }
#pragma unroll
  for (int t = 0; t < GDN_SHORT; ++t) {
    if (t < T) {
      float kv = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[e] *= gt[t];
        kv = __builtin_fmaf(s[e], kv8[t][e], kv);
      }
      kv = row16_sum(kv);
      const float dlt = (vt[t] - kv) * bt[t];
      float o = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[e] = __builtin_fmaf(kv8[t][e], dlt, s[e]);
        o = __builtin_fmaf(s[e], qv[t][e], o);
      }
      o = row16_sum(o);
      if (live && (lane & 15) == 0) {
        const int64_t yi = (((int64_t)b * T + t) * Hv + hv) * Dv + row;
        if constexpr (Y_F32)
          ((float *)y)[yi] = o;
        else
          ((uint16_t *)y)[yi] = f32_to_bf16_rne(o);
      }
    }
  }
  if (live) {
    *(float4 *)(st_out + so) = make_float4(s[0], s[1], s[2], s[3]);
    *(float4 *)(st_out + so + 4) = make_float4(s[4], s[5], s[6], s[7]);
  }
}

}  // namespace

template <bool IN, bool YF>
static void launch_gdn_t(const GdnArgs &a, unsigned grid, hipStream_t st) {
  if (a.T <= GDN_SHORT)
    hipLaunchKernelGGL((gdn_short_kernel<IN, YF>), dim3(grid), dim3(256), 0, st, a.T, a.Hk, a.Hv, a.Dv,
                       (int)a.beta_f32, a.state_in, a.q, a.k, a.v, a.g, a.beta, a.state_out, a.y);
  else if (a.T <= GDN_TB)
    hipLaunchKernelGGL((gdn_kernel<IN, YF, true>), dim3(grid), dim3(256), 0, st, a.q, a.k, a.v, a.g, a.beta,
                       (int)a.beta_f32, a.state_in, a.state_out, a.y, a.T, a.Hk, a.Hv, a.Dv);
  else
    hipLaunchKernelGGL((gdn_kernel<IN, YF, false>), dim3(grid), dim3(256), 0, st, a.q, a.k, a.v, a.g, a.beta,
                       (int)a.beta_f32, a.state_in, a.state_out, a.y, a.T, a.Hk, a.Hv, a.Dv);
}

hipError_t launch_gdn(const GdnArgs &a, hipStream_t st) {
  if (a.Dk != GDN_DK || a.Dv <= 0 || a.Dv % 8 != 0 || a.Hk <= 0 || a.Hv % a.Hk != 0 || a.T <= 0 || a.B <= 0)
    return hipErrorInvalidValue;
  const int groups = (a.Dv + 15) / 16;
  const int64_t grid = (int64_t)a.B * a.Hv * groups;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  const unsigned g = (unsigned)grid;
  if (a.in_f32)
    a.y_f32 ? launch_gdn_t<true, true>(a, g, st) : launch_gdn_t<true, false>(a, g, st);
  else
    a.y_f32 ? launch_gdn_t<false, true>(a, g, st) : launch_gdn_t<false, false>(a, g, st);
  return hipGetLastError();
}

}  // namespace qmm
