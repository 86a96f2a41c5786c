// Internal launcher interface between the C ABI (qmm_api.cpp) and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace qmm {

enum Mode : int { MXFP8 = 0, NVFP4 = 1 };

constexpr int QMV_MAX_M = 8;  // rows of x served by the decode (GEMV / skinny) kernels

// Where the decode kernels write output row r of y[M, N]: one bf16 array [M, N],
// or (a grouped call: several weight matrices of one K that share x and lie back
// to back in memory, run as one matrix) up to 4 arrays, row r in [lo_i, lo_(i+1))
// going to array i, an [M, n_i] row-major array, at row r - lo_i.
struct YOut {
  uint16_t *y0, *y1, *y2, *y3;
  int lo1, lo2, lo3;   // first row of parts 1..3 (INT32_MAX when absent)
  int n0, n1, n2, n3;  // rows of each part
  __host__ __device__ __forceinline__ uint16_t *at(int m, int r) const {
    if (r >= lo3) return y3 + (int64_t)m * n3 + (r - lo3);
    if (r >= lo2) return y2 + (int64_t)m * n2 + (r - lo2);
    if (r >= lo1) return y1 + (int64_t)m * n1 + (r - lo1);
    return y0 + (int64_t)m * n0 + r;
  }
};

// The parts of a grouped call's output (host side): part i has rows[i] rows.
struct QmmParts {
  int n;           // 1..4
  void *y[4];
  int rows[4];
};

struct QmmArgs {
  int mode;        // 0 = mxfp8, 1 = nvfp4
  bool x_f32;      // x (and y) float32 instead of bfloat16
  int M, N, K;     // y[M, N] = x[M, K] @ deq(W[N, K]).T
  const void *x;
  const uint8_t *w;  // packed rows, K*bits/8 bytes each
  const uint8_t *s;  // scale bytes, K/group per row
  void *y;
  const QmmParts *parts = nullptr;  // a grouped call's outputs (then y is unused)
  // The scales already in the prefill GEMMs' tile-major layout (the repack of
  // launch_repack_scales), or null: the GEMM then repacks them into its workspace.
  const uint32_t *s_tiled = nullptr;
  // mxfp8 prefill: x is already split into this call's workspace (the previous call on the
  // stream split the same x with the same M and K into the same workspace, for the same
  // kernel family: gemm_mxfp8_split_layout_of of both calls agree), so the split is skipped.
  bool x_split_ready = false;
};

// The output descriptor of a call: y as one part, or the grouped call's parts.
inline YOut yout_of(const QmmArgs &a) {
  YOut o{(uint16_t *)a.y, nullptr, nullptr, nullptr, INT32_MAX, INT32_MAX, INT32_MAX, a.N, 0, 0, 0};
  if (!a.parts) return o;
  const QmmParts &p = *a.parts;
  uint16_t **ys[4] = {&o.y0, &o.y1, &o.y2, &o.y3};
  int *los[4] = {nullptr, &o.lo1, &o.lo2, &o.lo3};
  int *ns[4] = {&o.n0, &o.n1, &o.n2, &o.n3};
  int lo = 0;
  for (int i = 0; i < p.n && i < 4; ++i) {
    *ys[i] = (uint16_t *)p.y[i];
    if (i > 0) *los[i] = lo;
    *ns[i] = p.rows[i];
    lo += p.rows[i];
  }
  return o;
}

// Whether the decode kernels that take a YOut serve these arguments (the grouped
// call's one-launch path; other shapes run one call per matrix).
bool qmv_parts_ok(const QmmArgs &a);
bool qmv_mfma_parts_ok(const QmmArgs &a);

bool qmv_fast_ok(const QmmArgs &a);
hipError_t launch_qmv(const QmmArgs &a, hipStream_t st);
hipError_t launch_qmv_generic(const QmmArgs &a, hipStream_t st);
// Decode GEMV on the scaled MFMA (K = 5120; nvfp4 M <= 2, mxfp8 M <= 4, bf16 x).
bool qmv_mfma_ok(const QmmArgs &a);
hipError_t launch_qmv_mfma(const QmmArgs &a, hipStream_t st);
bool qmv_mfma_mlp_ok(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up);
hipError_t launch_qmv_mfma_mlp(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st);
bool qmv_mlp_ok(const QmmArgs &a);
hipError_t launch_qmv_mlp(const QmmArgs &a, const uint8_t *w_up, const uint8_t *s_up, hipStream_t st);
hipError_t launch_silu_mul(const void *g, const void *u, void *h, int64_t n, bool f32, hipStream_t st);

// Prefill GEMM (M > QMV_MAX_M, and 5-8 rows the decode MFMA kernels do not take: qmm_on_decode).
bool gemm_ok(const QmmArgs &a);
hipError_t launch_gemm(const QmmArgs &a, hipStream_t st);

// mxfp8 prefill on the scaled fp8 MFMA (bf16 x split into E4M3 hi + lo).
bool gemm_mxfp8_ok(const QmmArgs &a);
size_t gemm_mxfp8_workspace(const QmmArgs &a);
// The layout launch_gemm_mxfp8 splits x into (0: row-major, 1: pre-tiled for the pipelined
// kernel); two calls may share one split only where this agrees.
int gemm_mxfp8_split_layout_of(const QmmArgs &a);
hipError_t launch_gemm_mxfp8(const QmmArgs &a, void *workspace, hipStream_t st);
bool gemm_nvfp4_ok(const QmmArgs &a);
size_t gemm_nvfp4_workspace(const QmmArgs &a);
hipError_t launch_gemm_nvfp4(const QmmArgs &a, void *workspace, hipStream_t st);

// The prefill GEMMs' scale layout: for each 256-row tile and each dword d of a row's
// nb scale bytes, 256 consecutive dwords (one per row).  tiled_scales_bytes(N, nb) bytes.
size_t tiled_scales_bytes(int64_t N, int nb);
hipError_t launch_repack_scales(const uint8_t *s, int64_t N, int nb, uint32_t *out, hipStream_t st);
// Whether the prefill GEMM for these arguments reads tile-major scales (and how many
// scale bytes per row it repacks): 0 when it reads them as stored.
int gemm_tiled_scale_bytes_per_row(const QmmArgs &a);

// Whether a call runs on the decode kernels (x of at most QMV_MAX_M rows, and x of up to
// 16 rows where the MFMA decode kernels take it: mxfp8 on the scaled MFMA, nvfp4 at
// K = 5120 / 6144 from 5 rows on the dequantizing bf16-MFMA kernel) rather than a prefill GEMM.  x of
// 5-8 rows that the MFMA decode kernels do not take (nvfp4 at K = 10240 / 17408; mxfp8 at
// K = 17408 from 6 rows) runs on the pipelined GEMM's split tiles when the matrix is tall:
// the other decode kernel is the unpacking GEMV, whose work grows with every row
// (N = 17408, K = 5120, nvfp4: 40-62 us at 5-8 rows against 25 us; N = 5120, K = 17408,
// mxfp8: 50-61 us against 47 us).
inline bool qmm_on_decode(const QmmArgs &a) {
  // (x of 9-16 rows on the MFMA decode kernels, where they take the shape)
  if (a.M > QMV_MAX_M) return a.M <= 16 && qmv_mfma_ok(a);
  if (a.M <= 4 || a.N < 4096 || qmv_mfma_ok(a) || ((uintptr_t)a.x | (uintptr_t)a.w) & 15) return true;
  if (a.mode == MXFP8) return !(gemm_mxfp8_ok(a) && a.K % 128 == 0 && ((uintptr_t)a.s & 3) == 0);
  return !gemm_nvfp4_ok(a);
}

// dequant: out [N, K] float32 (out_f32) or bfloat16.
hipError_t launch_dequant(int mode, const uint8_t *w, const uint8_t *s, int64_t N, int64_t K, void *out,
                          bool out_f32, hipStream_t st);
// quantize: in [N, K] float32 (in_f32) or bfloat16 -> packed words + scale bytes.
hipError_t launch_quantize(int mode, const void *in, bool in_f32, int64_t N, int64_t K, uint32_t *wq, uint8_t *s,
                           hipStream_t st);

// Gated-delta recurrence (the reference's packed GDN kernel, src/model.zig:284-319).
struct GdnArgs {
  int B, T, Hk, Hv, Dk, Dv;
  bool in_f32;    // q, k, v float32 (else bfloat16)
  bool beta_f32;  // beta float32 (else bfloat16)
  bool y_f32;     // y float32 (else bfloat16)
  const void *q, *k, *v, *beta;
  const float *g, *state_in;
  float *state_out;
  void *y;
};
hipError_t launch_gdn(const GdnArgs &a, hipStream_t st);
// The chunked form on the f32 MFMA, for long T: a per-chunk prep kernel writes its
// matrices to `workspace` (gdn_chunked_workspace bytes), a scan kernel runs the chunks.
constexpr int GDN_CHUNKED_MIN_T = 96;
bool gdn_chunked_ok(const GdnArgs &a);
size_t gdn_chunked_workspace(const GdnArgs &a);
hipError_t launch_gdn_chunked(const GdnArgs &a, void *workspace, hipStream_t st);
// The chunked form with its workspace in a static per-GPU array (no allocation): the
// array's size, whether a call's shape fits it (one batch's value heads x one chunk
// must), and the launch (several launches when the call's workspace exceeds the array).
size_t gdn_noalloc_scratch_bytes();
bool gdn_noalloc_fits(const GdnArgs &a);
hipError_t launch_gdn_chunked_noalloc(const GdnArgs &a, hipStream_t st);

// Zero-fill `bytes` of device memory.
hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t st);

// Compute units of the current device, cached per device (0, with the HIP error
// cleared, when no device answers: the caller's launch then reports the failure).
int device_cu_count();
// Raise a kernel's dynamic-LDS limit to `bytes` once per device.  `done` is the call
// site's own mask of devices already set (one bit per device id below 64; higher ids
// set it on every call).  Safe from several host threads: the attribute call is
// idempotent and the mask is atomic.
hipError_t ensure_dynamic_lds(std::atomic<uint64_t> &done, const void *kernel, int bytes);

// Dense bf16 y[M, N] = x[M, K] @ w[N, K].T (fp32 accumulate, RNE).
hipError_t launch_linear_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y, int M, int N, int K,
                              hipStream_t st);

}  // namespace qmm
