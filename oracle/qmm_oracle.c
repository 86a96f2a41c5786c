/*
 * qmm_oracle.c -- CPU restatement of mlx-runner's quantized linear layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only the test suite,
 * the smoke entry point and the benchmark's CPU-baseline leg load it.  The
 * product path (the HIP library) never links, loads or calls it.
 *
 * What it restates (reference paths are relative to the mlx-runner checkout):
 *   - mlx_quantized_matmul  src/mlx.zig:265, called by qlinear src/model.zig:244-260
 *       y[m,n] = sum_k x[m,k] * deq(W)[n,k]   (transpose_w = true, no biases)
 *   - mlx_dequantize        src/mlx.zig:274, used src/model.zig:1593 (dtype f32)
 *   - mlx_quantize          src/mlx.zig:278, used src/model.zig:1577
 *   - mode/group/bits pairs src/weights.zig:37-55 (mxfp8 = (32, 8), nvfp4 = (16, 4))
 *
 * The arithmetic lives in MLX 0.32.2 + mlx-c (third party, not vendored, not
 * importable here).  The formats are restated from their published
 * definitions:
 *   - OCP Microscaling Formats (MX) v1.0: E4M3 ("fn": no inf, S.1111.111 is
 *     NaN, max 448), E8M0 (2^(X-127), 0xFF is NaN), E2M1 {0,.5,1,1.5,2,3,4,6},
 *     MXFP8 = 32 E4M3 elements sharing one E8M0 scale.
 *   - NVFP4 = 16 E2M1 elements sharing one E4M3 scale; the per-tensor global
 *     scale is absent here (the reference passes a null global_scale,
 *     src/model.zig:1577, :1593), i.e. it is 1.
 *   - Packing (assumption, unpinned by the reference): element k of a row sits
 *     at byte k%4 of uint32 word k/4 (mxfp8) or nibble k%8 of word k/8
 *     (nvfp4), least significant first.  Scales are U8 [N, K/group].
 *   - Quantizer rounding (assumption, unpinned): mxfp8 follows the OCP MX v1.0
 *     reference rule (shared exponent floor(log2(amax)) - 8, elements RNE to
 *     E4M3 saturating at 448); nvfp4 scale = RNE_E4M3(amax / 6), elements
 *     RNE (ties to even code) to E2M1 of x / scale, saturating at 6.  Every
 *     rounding decision is made by exact comparisons.
 *   - Special values in quantized_matmul (assumption, unpinned): the
 *     dequantized weight elem * scale is taken exactly (double holds every
 *     product, 448 * 2^127 included), so a weight whose f32 dequant would
 *     overflow still multiplies x as its true value (0 * it is 0, and a tiny x
 *     gives a finite result); a NaN element code (E4M3 S.1111.111) or a NaN
 *     scale (E8M0 0xFF, E4M3 S.1111.111) makes the weight NaN and so every
 *     output that sums over it; y is the exact sum rounded once to bf16
 *     (overflow to +-inf).  mlx_dequantize to f32 rounds the same exact value
 *     to f32 (overflow to +-inf).
 *
 * Build: see oracle/Makefile (gcc -O3, pthreads).  No GPU, no torch.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QMM_MODE_MXFP8 0
#define QMM_MODE_NVFP4 1

/* ------------------------------------------------------------------ */
/* scalar decoders (closed forms)                                      */
/* ------------------------------------------------------------------ */

/* OCP E4M3 (fn): bias 7; subnormal m/8 * 2^-6; S.1111.111 -> NaN. */
float oracle_e4m3_to_f32(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
  double v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    v = ldexp((double)m, -9);
  else
    v = ldexp((double)(8 + m), e - 10);
  return (float)(s ? -v : v);
}

/* OCP E8M0: 2^(X-127) for X in 0..254 (X = 0 is the f32 subnormal 2^-127); 0xFF -> NaN. */
float oracle_e8m0_to_f32(uint8_t b) {
  if (b == 0xFF) return NAN;
  return (float)ldexp(1.0, (int)b - 127);
}

/* OCP E2M1: bias 1; subnormal 0.5*m; codes 0..7 = {0,.5,1,1.5,2,3,4,6}, bit 3 = sign. */
float oracle_e2m1_to_f32(uint8_t nib) {
  int s = (nib >> 3) & 1, e = (nib >> 1) & 3, m = nib & 1;
  double v = (e == 0) ? 0.5 * m : ldexp(1.0 + 0.5 * m, e - 1);
  return (float)(s ? -v : v);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round a double to the nearest bf16 (ties to even), in one rounding step.
 * bf16: 8 significant bits, f32 exponent range, subnormal quantum 2^-133. */
uint16_t oracle_f64_to_bf16(double v) {
  if (isnan(v)) return 0x7FC0;
  if (v == 0.0) return signbit(v) ? 0x8000 : 0x0000;
  int e;
  frexp(v, &e); /* |v| in [2^(e-1), 2^e) */
  int q = e - 1 - 7;
  if (q < -133) q = -133;
  double r = ldexp(nearbyint(ldexp(v, -q)), q); /* exact scaling, RNE */
  if (fabs(r) >= ldexp(1.0, 128)) return signbit(v) ? 0xFF80 : 0x7F80;
  float f = (float)r; /* exact: r has <= 8 significant bits in range */
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)(u >> 16);
}

uint16_t oracle_f32_to_bf16(float v) { return oracle_f64_to_bf16((double)v); }

/* Round a double to the nearest f32 (ties to even). */
static float f64_to_f32(double v) { return (float)v; }

/* ------------------------------------------------------------------ */
/* unpack + dequantize  (mlx_dequantize, src/mlx.zig:274)              */
/* ------------------------------------------------------------------ */

static inline uint8_t elem_code(int mode, const uint32_t *row, int64_t k) {
  if (mode == QMM_MODE_MXFP8) return (uint8_t)((row[k >> 2] >> (8 * (k & 3))) & 0xFF);
  return (uint8_t)((row[k >> 3] >> (4 * (k & 7))) & 0xF);
}

static inline float scale_value(int mode, uint8_t s) {
  return mode == QMM_MODE_MXFP8 ? oracle_e8m0_to_f32(s) : oracle_e4m3_to_f32(s);
}

static inline float elem_value(int mode, uint8_t c) {
  return mode == QMM_MODE_MXFP8 ? oracle_e4m3_to_f32(c) : oracle_e2m1_to_f32(c);
}

static inline int group_of(int mode) { return mode == QMM_MODE_MXFP8 ? 32 : 16; }
static inline int words_per_row(int mode, int64_t K) { return (int)(mode == QMM_MODE_MXFP8 ? K / 4 : K / 8); }

/* w[n,k] = elem(code) * scale, computed in double and rounded once to f32.
 * (For finite in-range values the product is exact in f32.) */
void oracle_dequant(int mode, const uint32_t *w, const uint8_t *s, int64_t N, int64_t K, float *out) {
  int g = group_of(mode);
  int64_t wpr = words_per_row(mode, K), spr = K / g;
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t *row = w + n * wpr;
    for (int64_t k = 0; k < K; ++k) {
      double v = (double)elem_value(mode, elem_code(mode, row, k)) * (double)scale_value(mode, s[n * spr + k / g]);
      out[n * K + k] = f64_to_f32(v);
    }
  }
}

/* w[n,k] = elem(code) * scale exactly, in double (no overflow: |w| <= 448 * 2^127). */
void oracle_dequant_f64(int mode, const uint32_t *w, const uint8_t *s, int64_t N, int64_t K, double *out) {
  int g = group_of(mode);
  int64_t wpr = words_per_row(mode, K), spr = K / g;
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t *row = w + n * wpr;
    for (int64_t k = 0; k < K; ++k)
      out[n * K + k] = (double)elem_value(mode, elem_code(mode, row, k)) * (double)scale_value(mode, s[n * spr + k / g]);
  }
}

/* Same, rounded to bf16 (the dtype=bfloat16 form of mlx_dequantize). */
void oracle_dequant_bf16(int mode, const uint32_t *w, const uint8_t *s, int64_t N, int64_t K, uint16_t *out) {
  int g = group_of(mode);
  int64_t wpr = words_per_row(mode, K), spr = K / g;
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t *row = w + n * wpr;
    for (int64_t k = 0; k < K; ++k) {
      double v = (double)elem_value(mode, elem_code(mode, row, k)) * (double)scale_value(mode, s[n * spr + k / g]);
      out[n * K + k] = oracle_f64_to_bf16(v);
    }
  }
}

/* ------------------------------------------------------------------ */
/* quantize (mlx_quantize, src/mlx.zig:278; rounding rule documented   */
/* above, an assumption)                                               */
/* ------------------------------------------------------------------ */

/* Nearest E4M3 code to a finite |v| (v >= 0), ties to even code, saturating at 448. */
static uint8_t e4m3_code_rne_sat(double v) {
  if (!(v > 0.0)) return 0;
  if (v >= 448.0) return 0x7E;
  int e;
  frexp(v, &e);           /* v in [2^(e-1), 2^e) */
  int q = (e - 1) - 3;    /* quantum for 3 mantissa bits */
  if (q < -9) q = -9;     /* subnormal quantum 2^-9 */
  double m = nearbyint(ldexp(v, -q)); /* exact scaling; RNE */
  double r = ldexp(m, q);
  if (r > 448.0) r = 448.0;
  /* encode r exactly */
  if (r < ldexp(1.0, -6)) return (uint8_t)(int)ldexp(r, 9); /* subnormal: m/8 * 2^-6 */
  int er;
  double fr = frexp(r, &er); /* r = fr * 2^er, fr in [0.5,1) */
  int E = er - 1 + 7;
  int M = (int)ldexp(fr * 2.0 - 1.0, 3);
  return (uint8_t)((E << 3) | M);
}

/* Nearest E2M1 code to |v| (v >= 0), ties to even code, saturating at 6. */
static uint8_t e2m1_code_rne_sat(double v) {
  /* representable magnitudes by code 0..7; midpoints between neighbours. */
  static const double mids[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0};
  int c = 0;
  while (c < 7 && v > mids[c]) ++c; /* c = lower neighbour when v == mids[c] */
  if (c < 7 && v == mids[c] && (c & 1)) c += 1; /* tie: the even code */
  return (uint8_t)c;
}

void oracle_quantize(int mode, const float *w, int64_t N, int64_t K, uint32_t *wq, uint8_t *s) {
  int g = group_of(mode);
  int64_t wpr = words_per_row(mode, K), spr = K / g;
  memset(wq, 0, sizeof(uint32_t) * N * wpr);
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t gi = 0; gi < spr; ++gi) {
      const float *v = w + n * K + gi * g;
      double amax = 0.0;
      for (int i = 0; i < g; ++i) amax = fmax(amax, fabs((double)v[i]));
      uint8_t sb;
      double sc;
      if (mode == QMM_MODE_MXFP8) {
        int X;
        if (amax == 0.0) {
          X = 0;
        } else {
          int e;
          frexp(amax, &e);           /* floor(log2(amax)) = e - 1 */
          X = (e - 1) - 8 + 127;     /* E4M3 emax = 8 */
          if (X < 0) X = 0;
          if (X > 254) X = 254;
        }
        sb = (uint8_t)X;
        sc = ldexp(1.0, X - 127);
      } else {
        /* RNE of amax/6 to E4M3, decided exactly: compare amax with 6 * midpoint. */
        {
          uint8_t best = 0;
          if (amax > 0.0) {
            /* candidate: the code whose value brackets amax/6 */
            double t = amax / 6.0;
            uint8_t c0 = e4m3_code_rne_sat(t);
            /* e4m3_code_rne_sat rounds t (already rounded to double) -- fix a
             * possible double-rounding by testing neighbours exactly. */
            double bestd = -1.0;
            for (int d = -1; d <= 1; ++d) {
              int c = (int)c0 + d;
              if (c < 0 || c > 0x7E) continue;
              double cv = (double)oracle_e4m3_to_f32((uint8_t)c);
              double diff = fabs(6.0 * cv - amax); /* exact: both <= 9 significant bits */
              if (bestd < 0.0 || diff < bestd || (diff == bestd && ((c & 1) == 0))) {
                bestd = diff;
                best = (uint8_t)c;
              }
            }
          }
          sb = best;
        }
        sc = (double)oracle_e4m3_to_f32(sb);
      }
      s[n * spr + gi] = sb;
      for (int i = 0; i < g; ++i) {
        int64_t k = gi * g + i;
        double x = (double)v[i];
        uint8_t code;
        if (mode == QMM_MODE_MXFP8) {
          double p = x / sc; /* exact: power-of-two scale */
          code = e4m3_code_rne_sat(fabs(p));
          if (signbit(p) && code != 0) code |= 0x80;
          wq[n * wpr + (k >> 2)] |= (uint32_t)code << (8 * (k & 3));
        } else {
          if (sc == 0.0) {
            code = 0;
          } else {
            /* compare |x| with mid * sc exactly (mid has <= 3, sc <= 4 significant bits) */
            static const double mids[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0};
            double ax = fabs(x);
            int c = 0;
            while (c < 7 && ax > mids[c] * sc) ++c;
            if (c < 7 && ax == mids[c] * sc && (c & 1)) c += 1;
            code = (uint8_t)c;
            if (signbit(x) && code != 0) code |= 0x8;
          }
          wq[n * wpr + (k >> 3)] |= (uint32_t)code << (4 * (k & 7));
        }
      }
    }
  }
}

/* exposed for the tests of the element rounding */
uint8_t oracle_e4m3_encode(double v) {
  uint8_t c = e4m3_code_rne_sat(fabs(v));
  return (signbit(v) && c != 0) ? (uint8_t)(c | 0x80) : c;
}
uint8_t oracle_e2m1_encode(double v) {
  uint8_t c = e2m1_code_rne_sat(fabs(v));
  return (signbit(v) && c != 0) ? (uint8_t)(c | 0x8) : c;
}

/* ------------------------------------------------------------------ */
/* quantized matmul (mlx_quantized_matmul, src/mlx.zig:265)            */
/* ------------------------------------------------------------------ */

#define X_BF16 0
#define X_F32 1
#define OUT_BF16 0
#define OUT_F32 1

typedef struct {
  int mode, x_dtype, out_kind, f32acc;
  const void *x;
  int64_t M, K, N;
  const uint32_t *w;
  const uint8_t *s;
  const int64_t *cols; /* optional subset of output columns n (NULL = all) */
  int64_t ncols;
  void *y; /* [M, ncols] */
  int64_t c0, c1;
  const double *xd; /* x as double [M, K] (exact) */
  const float *xf;  /* x as float  [M, K] (exact) */
} qmm_job;

/* Decode tables, filled from the closed forms above.  A product of two
 * decoded f32 values rounded once by an f32 multiply equals the double
 * product rounded once to f32, so table-driven dequant is bit-identical to
 * oracle_dequant. */
static float T_E4M3[256], T_E8M0[256], T_E2M1[16];
static pthread_once_t tables_once = PTHREAD_ONCE_INIT;
static void build_tables(void) {
  for (int i = 0; i < 256; ++i) {
    T_E4M3[i] = oracle_e4m3_to_f32((uint8_t)i);
    T_E8M0[i] = oracle_e8m0_to_f32((uint8_t)i);
  }
  for (int i = 0; i < 16; ++i) T_E2M1[i] = oracle_e2m1_to_f32((uint8_t)i);
}

/* The exact weights of one row (the parity path): every product of an element
 * and a scale is exact in double. */
static void dequant_row_f64(int mode, const uint32_t *row, const uint8_t *srow, int64_t K, double *out) {
  if (mode == QMM_MODE_MXFP8) {
    for (int64_t k = 0; k < K; ++k)
      out[k] = (double)T_E4M3[(row[k >> 2] >> (8 * (k & 3))) & 0xFF] * (double)T_E8M0[srow[k >> 5]];
  } else {
    for (int64_t k = 0; k < K; ++k)
      out[k] = (double)T_E2M1[(row[k >> 3] >> (4 * (k & 7))) & 0xF] * (double)T_E4M3[srow[k >> 4]];
  }
}

/* f32 weights (the CPU-baseline form): each product rounded once to f32. */
static void dequant_row_f32(int mode, const uint32_t *row, const uint8_t *srow, int64_t K, float *out) {
  if (mode == QMM_MODE_MXFP8) {
    for (int64_t k = 0; k < K; ++k) out[k] = T_E4M3[(row[k >> 2] >> (8 * (k & 3))) & 0xFF] * T_E8M0[srow[k >> 5]];
  } else {
    for (int64_t k = 0; k < K; ++k) out[k] = T_E2M1[(row[k >> 3] >> (4 * (k & 7))) & 0xF] * T_E4M3[srow[k >> 4]];
  }
}

static void *qmm_worker(void *arg) {
  qmm_job *j = (qmm_job *)arg;
  int g = group_of(j->mode);
  int64_t K = j->K, wpr = words_per_row(j->mode, K), spr = K / g;
  float *drow = (float *)malloc(sizeof(float) * (K + 16));
  double *ddrow = (double *)malloc(sizeof(double) * (K + 16));
  for (int64_t c = j->c0; c < j->c1; ++c) {
    int64_t n = j->cols ? j->cols[c] : c;
    if (j->f32acc)
      dequant_row_f32(j->mode, j->w + n * wpr, j->s + n * spr, K, drow);
    else
      dequant_row_f64(j->mode, j->w + n * wpr, j->s + n * spr, K, ddrow);
    for (int64_t m = 0; m < j->M; ++m) {
      double acc;
      if (j->f32acc) {
        /* fp32 accumulation (16 interleaved partial sums, then summed in
         * order): the CPU-baseline form. */
        const float *xr = j->xf + m * K;
        float part[16] = {0};
        int64_t k = 0;
        for (; k + 16 <= K; k += 16)
          for (int i = 0; i < 16; ++i) part[i] += xr[k + i] * drow[k + i];
        for (; k < K; ++k) part[0] += xr[k] * drow[k];
        float a = 0.0f;
        for (int i = 0; i < 16; ++i) a += part[i];
        acc = (double)a;
      } else {
        /* products of x (<= 24 significant bits) and an exact weight (<= 8) are
         * exact in double; sum in double. */
        const double *xr = j->xd + m * K;
        acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += xr[k] * ddrow[k];
      }
      if (j->out_kind == OUT_BF16)
        ((uint16_t *)j->y)[m * j->ncols + c] = oracle_f64_to_bf16(acc);
      else
        ((float *)j->y)[m * j->ncols + c] = f64_to_f32(acc);
    }
  }
  free(drow);
  free(ddrow);
  return NULL;
}

/*
 * y[m, c] = sum_k x[m,k] * deq(W)[cols[c], k]  for c < ncols (cols == NULL: all N).
 * f32acc = 0: exact weights, double accumulation rounded once (the parity oracle).
 * f32acc = 1: f32 weights, fp32 accumulation in K order (the CPU baseline).
 * threads: worker threads splitting the output columns.
 */
int oracle_qmm(int mode, int x_dtype, const void *x, int64_t M, int64_t K, const uint32_t *w, const uint8_t *s,
               int64_t N, const int64_t *cols, int64_t ncols, int out_kind, void *y, int f32acc, int threads) {
  pthread_once(&tables_once, build_tables);
  if (!cols) ncols = N;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if ((int64_t)threads > ncols) threads = ncols > 0 ? (int)ncols : 1;
  double *xd = NULL;
  float *xf = NULL;
  if (f32acc) {
    xf = (float *)malloc(sizeof(float) * (M * K + 1));
    for (int64_t i = 0; i < M * K; ++i)
      xf[i] = x_dtype == X_BF16 ? oracle_bf16_to_f32(((const uint16_t *)x)[i]) : ((const float *)x)[i];
  } else {
    xd = (double *)malloc(sizeof(double) * (M * K + 1));
    for (int64_t i = 0; i < M * K; ++i)
      xd[i] = x_dtype == X_BF16 ? (double)oracle_bf16_to_f32(((const uint16_t *)x)[i]) : (double)((const float *)x)[i];
  }
  pthread_t tid[256];
  qmm_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    qmm_job *j = &jobs[t];
    j->mode = mode;
    j->x_dtype = x_dtype;
    j->out_kind = out_kind;
    j->f32acc = f32acc;
    j->x = x;
    j->M = M;
    j->K = K;
    j->N = N;
    j->w = w;
    j->s = s;
    j->cols = cols;
    j->ncols = ncols;
    j->y = y;
    j->c0 = ncols * t / threads;
    j->c1 = ncols * (t + 1) / threads;
    j->xd = xd;
    j->xf = xf;
  }
  if (threads == 1) {
    qmm_worker(&jobs[0]);
  } else {
    for (int t = 0; t < threads; ++t) pthread_create(&tid[t], NULL, qmm_worker, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  }
  free(xd);
  free(xf);
  return 0;
}
