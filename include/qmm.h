/*
 * qmm.h -- C ABI of the MI355X (gfx950) quantized linear layer.
 *
 * Drop-in replacement for the mlx-c entry points that mlx-runner's quantized
 * linear path binds (reference paths relative to the mlx-runner checkout):
 *
 *   mlx_quantized_matmul   src/mlx.zig:265   -> qmm_quantized_matmul
 *   mlx_dequantize         src/mlx.zig:274   -> qmm_dequantize
 *   mlx_quantize           src/mlx.zig:278   -> qmm_quantize
 *   mlx_array / mlx_stream src/mlx.zig:10-11 -> qmm_array / qmm_stream
 *   mlx_optional_int       src/mlx.zig:41-51 -> qmm_optional_int
 *   mlx_dtype numbering    src/mlx.zig:21-36 -> qmm_dtype
 *   error latch            src/mlx.zig:719-868 -> qmm_set_error_handler, qmm_check_error, ...
 *   check + fault counter  src/mlx.zig:545-595 -> qmm_fault_arm, qmm_op_count
 *   WeightMap / QuantSpec  src/weights.zig:37-352 -> qmm_weights_* , qmm_infer_quant_spec_json
 *   namedLinearQ / qlinear src/model.zig:213-260 -> qmm_named_linear_q
 *
 * Conventions (same as mlx-c): every op returns 0 on success and non-zero on
 * failure; a failure also latches its message (first error wins) for the
 * next qmm_check_error().  Results are returned through an out-handle the
 * caller owns and frees with qmm_array_free; inputs are borrowed.  Ops are
 * eager and stream-ordered: a result is valid once its stream is synchronized,
 * and inputs must stay alive until then.
 *
 * All device memory is HBM on the current HIP device.  No torch types appear
 * in this interface.
 */
#ifndef QMM_H
#define QMM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- handles (opaque, one pointer wide, as mlx_array / mlx_stream) ---- */
typedef struct qmm_array_ { void *ctx; } qmm_array;
typedef struct qmm_stream_ { void *ctx; } qmm_stream;
typedef struct qmm_vector_array_ { void *ctx; } qmm_vector_array;
typedef struct qmm_weight_map_ { void *ctx; } qmm_weight_map;

/* dtype codes follow mlx_dtype (src/mlx.zig:21-36). */
typedef enum {
  QMM_BOOL = 0, QMM_UINT8 = 1, QMM_UINT16 = 2, QMM_UINT32 = 3, QMM_UINT64 = 4,
  QMM_INT8 = 5, QMM_INT16 = 6, QMM_INT32 = 7, QMM_INT64 = 8,
  QMM_FLOAT16 = 9, QMM_FLOAT32 = 10, QMM_FLOAT64 = 11, QMM_BFLOAT16 = 12, QMM_COMPLEX64 = 13
} qmm_dtype;

typedef struct { int value; bool has_value; } qmm_optional_int;         /* src/mlx.zig:41-51 */
typedef struct { qmm_dtype value; bool has_value; } qmm_optional_dtype; /* mlx_optional_dtype */

/* ---- arrays ---- */
/* Empty handle (mlx_array_new). */
qmm_array qmm_array_new(void);
/* New HBM array holding a copy of host `data` (mlx_array_new_data).  NULL ctx on failure. */
qmm_array qmm_array_new_data(const void *data, const int *shape, int dim, qmm_dtype dtype);
/* Wrap an existing device buffer without copying or taking ownership.  No
 * mlx-c counterpart: lets a caller hand HBM it already owns (e.g. a loader's
 * buffer) to the ops.  The buffer must outlive the handle. */
qmm_array qmm_array_new_device(void *device_ptr, const int *shape, int dim, qmm_dtype dtype);
int qmm_array_free(qmm_array a);                                  /* mlx_array_free */
size_t qmm_array_ndim(qmm_array a);                               /* mlx_array_ndim */
const int *qmm_array_shape(qmm_array a);                          /* mlx_array_shape */
qmm_dtype qmm_array_dtype(qmm_array a);                           /* mlx_array_dtype */
size_t qmm_array_size(qmm_array a);                               /* mlx_array_size */
size_t qmm_array_nbytes(qmm_array a);                             /* mlx_array_nbytes */
void *qmm_array_data_device(qmm_array a);                         /* device pointer */
/* Copy the array to host memory after its stream's pending work (the
 * eval + mlx_array_data_* step).  Returns non-zero on size mismatch. */
int qmm_array_to_host(void *dst, size_t nbytes, qmm_array a, qmm_stream s);

/* ---- streams ---- */
qmm_stream qmm_default_gpu_stream_new(void);      /* gpuStream, src/mlx.zig:425-427 (null HIP stream) */
qmm_stream qmm_stream_new_from_hip(void *hip_stream); /* wrap a caller's hipStream_t (borrowed) */
int qmm_stream_free(qmm_stream s);
int qmm_synchronize(qmm_stream s);                /* mlx_synchronize */

/* ---- ops ---- */
/* y = x @ deq(w).T  (src/mlx.zig:265; called by qlinear, src/model.zig:244-260).
 *  x: bf16 or f32 [..., M, K]; w: uint32 [N, K*bits/32]; scales: uint8 [N, K/group];
 *  biases must be the null handle; transpose_w must be true;
 *  group_size / bits: optional, default by mode (mxfp8 -> 32/8, nvfp4 -> 16/4), else must match;
 *  mode: "mxfp8" | "nvfp4".  y: [..., M, N] in x's dtype (fp32 accumulation, RNE).
 * If *res already holds an array of exactly the output shape and dtype its
 * buffer is written in place (no allocation); otherwise *res is replaced by a
 * new array.  Prefill calls (M > 8) read the scales in a tile-major copy that the
 * library makes at the first such call with this scales handle (not while the
 * stream is being captured) and frees with the handle: as with mlx arrays, the
 * contents behind a handle must not change while it lives.  The copy holds
 * round_up(N, 256) * K / group bytes of device memory (1/8 of the packed weight
 * bytes for nvfp4, 1/32 for mxfp8).  It is complete on the device before any call
 * uses it: the first prefill call with a handle waits for its stream once, after
 * which calls on any stream or thread read the copy with no further ordering.
 * Freeing a handle that holds a copy waits for the device (hipFree).
 * Prefill calls also take per-call scratch from a workspace kept per device and
 * stream (see qmm_gdn_recurrence); a graph captured on a stream uses that stream's
 * workspace when it is large enough, so replays of it must not overlap eager calls
 * on the capture stream (replay on that stream, or synchronize in between). */
int qmm_quantized_matmul(qmm_array *res, qmm_array x, qmm_array w, qmm_array scales, qmm_array biases,
                         bool transpose_w, qmm_optional_int group_size, qmm_optional_int bits,
                         const char *mode, qmm_stream s);

/* res[i] = x @ deq(w[i]).T for i < n (1 <= n <= 4): projections of one x with the
 * same K and mode, each argument as in qmm_quantized_matmul (res[i] written in
 * place when it holds an array of the output shape).  Replaces n consecutive
 * qlinear calls on one x: the GDN layer's in_proj_qkv / z / b / a
 * (src/model.zig:1066-1074) and attention's q / k / v (:929-944).  When the
 * matrices lie back to back in memory, and so do their scales (in any order;
 * qmm_weights_load places each layer's groups so), with bfloat16 x, one kernel
 * runs over them as one matrix: the decode kernel at M <= 4, the prefill GEMM at
 * the sizes it takes (the stacked scales are then repacked per call); otherwise one
 * call per matrix.  Either way res[i] meets the bar of
 * qmm_quantized_matmul(x, w[i], scales[i]); the one launch picks its kernel and tiling
 * by the total row count, which can differ from the single call's choice, so the bf16
 * roundings of the two may differ. */
int qmm_quantized_matmul_group(qmm_array *res, size_t n, qmm_array x, const qmm_array *w, const qmm_array *scales,
                               qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                               qmm_stream s);

/* deq(w) as [N, K] of `dtype` (default bfloat16; float32 and bfloat16 supported)
 * (src/mlx.zig:274).  biases and global_scale must be null handles. */
int qmm_dequantize(qmm_array *res, qmm_array w, qmm_array scales, qmm_array biases,
                   qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                   qmm_array global_scale, qmm_optional_dtype dtype, qmm_stream s);

/* [packed uint32, scales uint8] from a bf16/f32 [N, K] matrix (src/mlx.zig:278).
 * Rounding: mxfp8 shared exponent floor(log2(amax)) - 8, elements RNE to E4M3
 * saturating at 448; nvfp4 scale RNE_E4M3(amax/6), elements RNE to E2M1,
 * saturating at 6.  global_scale must be the null handle. */
int qmm_quantize(qmm_vector_array *res, qmm_array w, qmm_optional_int group_size, qmm_optional_int bits,
                 const char *mode, qmm_array global_scale, qmm_stream s);

/* The gated-delta (GDN) recurrence of mlx-runner's linear-attention layers: the
 * packed kernel gdnKernelRun launches (src/model.zig:284-319, source
 * src/gdn_packed.metal), with the shape rules of fusedEligible (:322-329).
 * q, k [B, T, Hk, Dk=128] and v [B, T, Hv, Dv] (Dv % 8 == 0, Hv % Hk == 0), all
 * bfloat16 or all float32; g [B, T, Hv] float32; beta [B, T, Hv] bfloat16 or
 * float32; state [B, Hv, Dv, Dk] float32.  Value head hv uses key head
 * hv / (Hv / Hk).  Per step: S *= g; dlt = (v - S k) beta; S += dlt k^T; y = S q.
 * Results: y [B, T, Hv, Dv] in y_dtype (bfloat16 RNE or float32) and the final
 * state [B, Hv, Dv, Dk] float32.  state_out may be the state's own handle (the
 * update is then in place).  q, k and state must be 16-byte aligned.  g must lie
 * in [0, 1] (the model's decays exp(-softplus(.) * A) do): a NaN g gives NaN in y
 * from its step on (in the chunked form below, from the first step of its 64-step
 * chunk) and in the state; a negative g gives NaN likewise in the chunked form.
 * From T = 96 (with Dv % 16 == 0) the steps run in chunks of 64 as matrix products
 * (the same recurrence to f32 rounding for g in [0, 1]), with a workspace of
 * B * Hv * ceil(T / 64) * 33 KB: the library's grow-only workspace of the stream
 * (one per device and stream, kept until the process ends), or, while the stream
 * is being captured into a graph and that is too small, an allocation made on the
 * stream and released after the call's kernels.  The prefill GEMMs of
 * qmm_quantized_matmul (M > 8) take theirs the same way. */
int qmm_gdn_recurrence(qmm_array *y, qmm_array *state_out, qmm_array q, qmm_array k, qmm_array v, qmm_array g,
                       qmm_array beta, qmm_array state, qmm_dtype y_dtype, qmm_stream s);

/* qmm_gdn_recurrence without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Arguments and results as in
 * qmm_gdn_recurrence, except that *y and *state_out must already hold arrays of the
 * results' shapes and dtypes ([B, T, Hv, Dv] y_dtype; [B, Hv, Dv, Dk] float32, which
 * may be the state's own handle); otherwise the call fails and allocates nothing.
 * The chunked form's workspace (T >= 96) is a 64 MiB array in the library, one per
 * GPU, held until the process ends: a call whose workspace is larger runs as several
 * launches (groups of whole batches, or runs of whole 64-step chunks of one batch),
 * with results identical bit for bit to one launch; Hv above 2016 value heads (one
 * 64-step chunk of one batch over all of them exceeds the array) is rejected.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and give wrong results. */
int qmm_gdn_recurrence_noalloc(qmm_array *y, qmm_array *state_out, qmm_array q, qmm_array k, qmm_array v,
                               qmm_array g, qmm_array beta, qmm_array state, qmm_dtype y_dtype, qmm_stream s);

/* silu(g) * u element-wise, with mlx-runner's per-op roundings in the arrays' dtype
 * (bfloat16 or float32): sg = sigmoid(g), sl = g * sg, h = sl * u, each rounded
 * (silu src/model.zig:405-415, mul :451-456).  g and u must have equal shapes. */
int qmm_silu_mul(qmm_array *res, qmm_array g, qmm_array u, qmm_stream s);

/* h = silu(x @ deq(Wg).T) * (x @ deq(Wu).T): the first three ops of mlpForwardQ
 * (src/model.zig:905-913) in one call, same arguments as qmm_quantized_matmul for
 * each projection.  Decode shapes (M <= 4) run one fused kernel (the gate and up
 * rows of an output in one wave, the activation in its epilogue); the result
 * equals quantized_matmul x 2 + silu_mul. */
int qmm_mlp_gate_up_silu(qmm_array *res, qmm_array x, qmm_array w_gate, qmm_array s_gate, qmm_array w_up,
                         qmm_array s_up, qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                         qmm_stream s);

qmm_vector_array qmm_vector_array_new(void);
int qmm_vector_array_free(qmm_vector_array v);
size_t qmm_vector_array_size(qmm_vector_array v);
int qmm_vector_array_get(qmm_array *res, qmm_vector_array v, size_t idx); /* new handle, caller frees */

/* ---- errors (src/mlx.zig:719-868) ---- */
typedef void (*qmm_error_handler_func)(const char *msg, void *data);
/* Install a handler called with every error message (after it is latched). */
int qmm_set_error_handler(qmm_error_handler_func handler, void *data, void (*dtor)(void *));
bool qmm_error_pending(void);
/* Memory-class message? (hipErrorOutOfMemory and allocation failures) */
bool qmm_error_is_memory(const char *msg);
/* Name of the class the next check would raise ("OutOfMemory" / "MlxFailure"), or NULL; does not consume. */
const char *qmm_peek_error_name(void);
/* Consume the latched message into buf; returns its length, or -1 if none. */
int qmm_take_error(char *buf, size_t len);
/* Checkpoints: 0 = no error, QMM_ERR_OOM, QMM_ERR_FAILURE; consume the latch.
 * An error the HIP runtime holds for the calling thread (hipGetLastError) is
 * latched first, except hipErrorNotReady (a query's answer) and hipErrorNoDevice.
 * Every op that launches work clears such a leftover runtime error when it starts,
 * so an op reports only its own failures, not one the caller's code left behind.  They do not wait for the device: an error of work still in
 * flight surfaces at the call that waits for it (qmm_synchronize,
 * qmm_array_to_host), which latches it, so call qmm_synchronize before a
 * checkpoint that must cover all enqueued work.
 * Env QMM_FAULT_CHUNK=<n> / QMM_FAULT_STEP=<n> latch a synthetic memory error at
 * the n-th call of qmm_check_error / qmm_check_error_decode (then disarm). */
#define QMM_ERR_OOM 1
#define QMM_ERR_FAILURE 2
int qmm_check_error(void);
int qmm_check_error_decode(void);
void qmm_latch_error_for_test(const char *msg);
void qmm_reset_faults_for_test(void);
/* Test fault injection at the op chokepoint (src/mlx.zig:562-595): the k-th
 * subsequent op that would succeed reports failure instead (its outputs stay
 * valid and freeable).  arm(0) disarms. */
void qmm_fault_arm(uint64_t k);
bool qmm_fault_did_fire(void);
uint64_t qmm_op_count(void);
/* Grouped calls (qmm_quantized_matmul_group) that ran as one kernel launch (diagnostics). */
uint64_t qmm_group_launch_count(void);
/* Bytes of device memory held by the tile-major scale copies of live scales handles
 * (see qmm_quantized_matmul; diagnostics, no mlx-c counterpart). */
uint64_t qmm_scale_copy_bytes(void);

/* ---- weights (src/weights.zig) ---- */
typedef enum { QMM_QUANT_NONE = 0, QMM_QUANT_MXFP8 = 1, QMM_QUANT_NVFP4 = 2 } qmm_quant_mode;
typedef struct { qmm_quant_mode mode; uint32_t group_size; uint32_t bits; } qmm_quant_spec;

/* Error codes of the loader / header checks (WeightsError, src/weights.zig:23-33). */
#define QMM_WE_BAD_INDEX_JSON 101
#define QMM_WE_BAD_HEADER 102
#define QMM_WE_UNSUPPORTED_DTYPE 103
#define QMM_WE_UNSUPPORTED_LAYOUT 104
#define QMM_WE_MISSING_TENSOR 105
#define QMM_WE_DUPLICATE_TENSOR 106
#define QMM_WE_NONSTANDARD_QUANT 107
#define QMM_WE_INCONSISTENT_QUANT 108
#define QMM_WE_AFFINE_UNSUPPORTED 109
#define QMM_WE_IO 110
#define QMM_WE_MISSING_WEIGHT 111

/* Parse + validate one safetensors header JSON (parseHeaderJson, src/weights.zig:70-121)
 * and infer the quant spec from it alone (inferQuantSpec, :130-185).  Host-only.
 * Returns 0 or a QMM_WE_* code; *n_tensors receives the tensor count. */
int qmm_infer_quant_spec_json(const char *json, size_t len, qmm_quant_spec *spec, size_t *n_tensors);
/* Header parse only. */
int qmm_parse_header_json(const char *json, size_t len, size_t *n_tensors);
/* Name remap (sanitizeName, :186-202): writes the kept name into out (NUL
 * terminated); returns 1 kept, 0 dropped, <0 if out is too small. */
int qmm_sanitize_name(const char *name, char *out, size_t out_len);

/* Load a sharded safetensors checkpoint (model.safetensors.index.json + shards)
 * into HBM, tensors copied raw from their data_offsets (WeightMap.load, :257-352).
 * The packed weights of each layer's linear_attn.in_proj_{qkv,z,b,a},
 * self_attn.{q,k,v}_proj and mlp.{gate,up}_proj are placed back to back in that
 * order (and their scales likewise) when every member is present and all but the
 * last are multiples of 256 bytes, for qmm_quantized_matmul_group. */
int qmm_weights_load(qmm_weight_map *res, const char *model_dir, qmm_stream s);
int qmm_weights_free(qmm_weight_map m);
/* Borrowed handle (do not free), or a NULL ctx when absent (WeightMap.get). */
qmm_array qmm_weights_get(qmm_weight_map m, const char *name);
size_t qmm_weights_count(qmm_weight_map m);
qmm_quant_spec qmm_weights_quant(qmm_weight_map m);

/* y = x @ W.T with the checkpoint's quantization honored (namedLinearQ,
 * src/model.zig:213-233): packed U32 + `<prefix>.scales` -> qmm_quantized_matmul
 * with the map's group/bits/mode; no scales and non-U32 weight -> dense bf16
 * linear (src/model.zig:200-211); U32 weight without scales or a name not ending
 * in ".weight" -> QMM_WE_MISSING_WEIGHT. */
int qmm_named_linear_q(qmm_array *res, qmm_weight_map m, qmm_array x, const char *name, qmm_stream s);
/* n <= 4 projections of one x by checkpoint name (layerLinearQ calls on one x,
 * src/model.zig:1066-1074 and :929-944): qmm_quantized_matmul_group when every
 * weight is packed with scales, else qmm_named_linear_q per name. */
int qmm_named_linear_q_group(qmm_array *res, size_t n, qmm_weight_map m, qmm_array x, const char *const *names,
                             qmm_stream s);
/* Dense y = x @ w.T for bf16 x [..., M, K] and bf16 w [N, K] (linear, src/model.zig:200-211). */
int qmm_linear(qmm_array *res, qmm_array x, qmm_array w, qmm_stream s);
/* mlpForwardQ (src/model.zig:905-915): down(silu(gate(x)) * up(x)) by checkpoint
 * names, in the reference's argument order (gate, down, up). */
int qmm_mlp_forward_q(qmm_array *res, qmm_weight_map m, qmm_array x, const char *gate_name, const char *down_name,
                      const char *up_name, qmm_stream s);

/* Library / device info. */
const char *qmm_version(void);
int qmm_device_info(char *buf, size_t len);

#ifdef __cplusplus
}
#endif
#endif /* QMM_H */
