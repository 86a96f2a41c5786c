// C ABI core: arrays, streams, error latch, op chokepoint, and the three ops
// mlx-runner's quantized linear path binds (src/mlx.zig:265, :274, :278).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qmm.h"
#include "qmm_internal.h"
#include "qmm_launch.h"

namespace qmm {

// ---------------------------------------------------------------- error latch (src/mlx.zig:719-868)
namespace {
std::mutex g_err_mtx;
std::atomic<bool> g_latched{false};
char g_err_buf[512];
size_t g_err_len = 0;
qmm_error_handler_func g_handler = nullptr;
void *g_handler_data = nullptr;
void (*g_handler_dtor)(void *) = nullptr;

// test fault counter at the op chokepoint (src/mlx.zig:562-595)
std::atomic<uint64_t> g_op_count{0};
uint64_t g_fault_remaining = 0;
bool g_fault_fired = false;

// env-armed checkpoint faults (MLX_SERVE_MLX_FAULT_CHUNK / _STEP analogues, src/mlx.zig:807-868)
struct FaultSite {
  const char *env;
  const char *msg;
  long long at = -1;  // -1: env not read yet
  unsigned long long seen = 0;
  long long target() {
    if (at >= 0) return at;
    at = 0;
    if (const char *p = std::getenv(env)) at = std::atoll(p) > 0 ? std::atoll(p) : 0;
    if (at > 0) std::fprintf(stderr, "[qmm] FAULT INJECTION armed: %s=#%lld\n", env, at);
    return at;
  }
  void maybe_fire() {
    long long t = target();
    if (t == 0) return;
    seen += 1;
    if ((long long)seen != t) return;
    at = 0;
    latch_error(msg);
  }
  void reset() {
    at = -1;
    seen = 0;
  }
};
FaultSite g_fault_chunk{"QMM_FAULT_CHUNK",
                        "[qmm] hipErrorOutOfMemory: out of memory (injected by QMM_FAULT_CHUNK)"};
FaultSite g_fault_step{"QMM_FAULT_STEP", "[qmm] hipErrorOutOfMemory: out of memory (injected by QMM_FAULT_STEP)"};
}  // namespace

void latch_error(const char *msg) {
  {
    std::lock_guard<std::mutex> lk(g_err_mtx);
    if (!g_latched.load(std::memory_order_acquire)) {  // first error wins
      size_t n = std::strlen(msg);
      if (n > sizeof(g_err_buf) - 1) n = sizeof(g_err_buf) - 1;
      std::memcpy(g_err_buf, msg, n);
      g_err_buf[n] = 0;
      g_err_len = n;
      g_latched.store(true, std::memory_order_release);
    }
  }
  if (g_handler)
    g_handler(msg, g_handler_data);
  else
    std::fprintf(stderr, "[qmm] %s\n", msg);
}

int fail(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  latch_error(buf);
  return 1;
}

// Latches a failed HIP call's error and clears the runtime's record of it, so that
// what the runtime still holds at a checkpoint is an error the library has not seen.
int fail_hip(hipError_t e, const char *what) {
  (void)hipGetLastError();
  return fail("[%s] %s: %s", what, hipGetErrorName(e), hipGetErrorString(e));
}

// Called at the start of every op that launches work: an error the HIP runtime still
// holds for this thread at that point comes from outside the op (a failed call in the
// caller's own code, a query's hipErrorNotReady).  The launch helpers read the runtime's
// last error after each launch, so such a leftover would make the op report a failure
// it did not have; clearing it first leaves each op reporting only its own.
void begin_op() { (void)hipGetLastError(); }

// The chokepoint every op returns through: counts ops and applies the armed test fault.
int finish(int rc) {
  g_op_count.fetch_add(1, std::memory_order_relaxed);
  if (rc != 0) return rc;
  if (g_fault_remaining != 0) {
    g_fault_remaining -= 1;
    if (g_fault_remaining == 0) {
      g_fault_fired = true;
      return 1;
    }
  }
  return 0;
}

// ---------------------------------------------------------------- arrays
size_t dtype_size(qmm_dtype d) {
  switch (d) {
    case QMM_BOOL: case QMM_UINT8: case QMM_INT8: return 1;
    case QMM_UINT16: case QMM_INT16: case QMM_FLOAT16: case QMM_BFLOAT16: return 2;
    case QMM_UINT32: case QMM_INT32: case QMM_FLOAT32: return 4;
    case QMM_UINT64: case QMM_INT64: case QMM_FLOAT64: case QMM_COMPLEX64: return 8;
  }
  return 0;
}

size_t Arr::size() const {
  size_t n = 1;
  for (int i = 0; i < ndim; ++i) n *= (size_t)shape[i];
  return n;
}

namespace {
bool g_pool_ready = false;
std::mutex g_pool_mtx;
void pool_init() {
  std::lock_guard<std::mutex> lk(g_pool_mtx);
  if (g_pool_ready) return;
  g_pool_ready = true;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();  // the op's own allocation reports the problem
    return;
  }
  hipMemPool_t pool;
  if (hipDeviceGetDefaultMemPool(&pool, dev) == hipSuccess) {
    uint64_t thr = UINT64_MAX;  // keep freed blocks cached for reuse
    (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &thr);
  }
}
}  // namespace

// Stream-ordered HBM allocation (cached by the device's default pool).
int alloc_device(void **p, size_t bytes, hipStream_t st) {
  pool_init();
  *p = nullptr;
  if (bytes == 0) bytes = 1;
  hipError_t e = hipMallocAsync(p, bytes, st);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail("[qmm::malloc] Unable to allocate %zu bytes: %s (out of memory)", bytes, hipGetErrorName(e));
  }
  return 0;
}

// ---------------------------------------------------------------- workspaces
// One grow-only workspace per (device, stream), for the per-call scratch of the
// prefill GEMMs and the chunked GDN form.  Calls on one stream are ordered, so they
// can share it; calls on different streams get different ones.  A buffer the stream
// outgrows stays allocated until the process ends: a graph captured earlier may
// still point at it.  Sizes are powers of two from 1 MiB, so what is kept is under
// twice the largest request.
namespace {
std::mutex g_ws_mtx;
std::map<std::pair<int, uintptr_t>, std::pair<void *, size_t>> g_ws;
}  // namespace

int workspace(hipStream_t st, size_t bytes, void **out, bool *transient) {
  *transient = false;
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "qmm::workspace");
  std::lock_guard<std::mutex> lk(g_ws_mtx);
  auto &ent = g_ws[{dev, (uintptr_t)st}];
  if (ent.first && ent.second >= bytes) {
    *out = ent.first;
    return 0;
  }
  // While the stream is being captured, growing would record an allocation into the
  // graph that the cache then keeps: take a transient allocation instead.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    cs = hipStreamCaptureStatusActive;  // unknown: the transient path is safe either way
  }
  if (cs != hipStreamCaptureStatusNone) {
    *transient = true;
    return alloc_device(out, bytes, st);
  }
  size_t cap = (size_t)1 << 20;
  while (cap < bytes) cap <<= 1;
  void *p = nullptr;
  if (alloc_device(&p, cap, st)) return 1;
  ent = {p, cap};
  *out = p;
  return 0;
}

Arr *new_arr(const int *shape, int dim, qmm_dtype dtype) {
  if (dim < 0 || dim > QMM_MAX_DIM) return nullptr;
  Arr *a = new Arr();
  a->ndim = dim;
  for (int i = 0; i < dim; ++i) a->shape[i] = shape[i];
  a->dtype = dtype;
  return a;
}

int alloc_arr(qmm_array *res, const std::vector<int> &shape, qmm_dtype dtype, hipStream_t st, Arr **out) {
  // Reuse the caller's array when it already has exactly this shape and dtype.
  Arr *cur = res ? (Arr *)res->ctx : nullptr;
  if (cur && cur->data && cur->dtype == dtype && cur->ndim == (int)shape.size()) {
    bool same = true;
    for (int i = 0; i < cur->ndim; ++i) same &= cur->shape[i] == shape[i];
    if (same) {
      *out = cur;
      return 0;
    }
  }
  Arr *a = new_arr(shape.data(), (int)shape.size(), dtype);
  if (!a) return fail("[qmm] array rank %zu exceeds %d", shape.size(), QMM_MAX_DIM);
  if (alloc_device(&a->data, a->nbytes(), st)) {
    delete a;
    return 1;
  }
  a->owned = true;
  a->alloc_stream = st;
  if (cur) release_arr(cur);
  res->ctx = a;
  *out = a;
  return 0;
}

// Bytes held by the tile-major scale copies of live handles (diagnostics).
static std::atomic<uint64_t> g_tiled_bytes{0};

void release_tiled(Arr *a) {
  if (!a || !a->tiled) return;
  // A plain allocation: hipFree waits for the device first, so work already queued on any
  // stream that reads the copy completes before it goes; no caller stream is involved.
  (void)hipFree(a->tiled);
  (void)hipGetLastError();
  g_tiled_bytes.fetch_sub(a->tiled_bytes, std::memory_order_relaxed);
  a->tiled = nullptr;
  a->tiled_bytes = 0;
}

void release_arr(Arr *a) {
  if (!a) return;
  if (a->owned && a->data) (void)hipFreeAsync(a->data, a->alloc_stream);
  release_tiled(a);
  delete a;
}

hipStream_t stream_of(qmm_stream s) { return s.ctx ? ((Stream *)s.ctx)->h : (hipStream_t)0; }

}  // namespace qmm

using namespace qmm;

// ================================================================ C ABI

extern "C" {

const char *qmm_version(void) { return "qmm-gfx950 0.1"; }

int qmm_device_info(char *buf, size_t len) {
  int dev = 0;
  hipDeviceProp_t p;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail("[qmm_device_info] no HIP device");
  }
  std::snprintf(buf, len, "%s %s CUs=%d clock_khz=%d mem_clock_khz=%d bus_bits=%d hbm_bytes=%zu l2=%d",
                p.name, p.gcnArchName, p.multiProcessorCount, p.clockRate, p.memoryClockRate, p.memoryBusWidth,
                (size_t)p.totalGlobalMem, p.l2CacheSize);
  return 0;
}

// ---------------- arrays
qmm_array qmm_array_new(void) { return qmm_array{nullptr}; }

qmm_array qmm_array_new_data(const void *data, const int *shape, int dim, qmm_dtype dtype) {
  Arr *a = new_arr(shape, dim, dtype);
  if (!a || dtype_size(dtype) == 0) {
    delete a;
    fail("[qmm_array_new_data] bad rank or dtype");
    return qmm_array{nullptr};
  }
  if (alloc_device(&a->data, a->nbytes(), (hipStream_t)0)) {
    delete a;
    return qmm_array{nullptr};
  }
  a->owned = true;
  a->alloc_stream = (hipStream_t)0;
  if (a->nbytes()) {
    hipError_t e = hipMemcpy(a->data, data, a->nbytes(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      fail_hip(e, "qmm_array_new_data");
      release_arr(a);
      return qmm_array{nullptr};
    }
  }
  return qmm_array{a};
}

qmm_array qmm_array_new_device(void *device_ptr, const int *shape, int dim, qmm_dtype dtype) {
  Arr *a = new_arr(shape, dim, dtype);
  if (!a || dtype_size(dtype) == 0) {
    delete a;
    fail("[qmm_array_new_device] bad rank or dtype");
    return qmm_array{nullptr};
  }
  for (int i = 0; i < dim; ++i)
    if (shape[i] < 0) {
      delete a;
      fail("[qmm_array_new_device] negative dimension");
      return qmm_array{nullptr};
    }
  a->data = device_ptr;
  a->owned = false;
  return qmm_array{a};
}

int qmm_array_free(qmm_array a) {
  release_arr((Arr *)a.ctx);
  return 0;
}
size_t qmm_array_ndim(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->ndim : 0; }
const int *qmm_array_shape(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->shape : nullptr; }
qmm_dtype qmm_array_dtype(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->dtype : QMM_BOOL; }
size_t qmm_array_size(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->size() : 0; }
size_t qmm_array_nbytes(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->nbytes() : 0; }
void *qmm_array_data_device(qmm_array a) { return a.ctx ? ((Arr *)a.ctx)->data : nullptr; }

int qmm_array_to_host(void *dst, size_t nbytes, qmm_array a, qmm_stream s) {
  Arr *x = (Arr *)a.ctx;
  if (!x) return finish(fail("[qmm_array_to_host] empty array"));
  if (nbytes != x->nbytes()) return finish(fail("[qmm_array_to_host] size %zu != array bytes %zu", nbytes, x->nbytes()));
  hipStream_t st = stream_of(s);
  hipError_t e = hipMemcpyAsync(dst, x->data, nbytes, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return finish(fail_hip(e, "qmm_array_to_host"));
  return finish(0);
}

// ---------------- streams
qmm_stream qmm_default_gpu_stream_new(void) {
  Stream *s = new Stream();
  s->h = (hipStream_t)0;
  return qmm_stream{s};
}
qmm_stream qmm_stream_new_from_hip(void *hip_stream) {
  Stream *s = new Stream();
  s->h = (hipStream_t)hip_stream;
  return qmm_stream{s};
}
int qmm_stream_free(qmm_stream s) {
  delete (Stream *)s.ctx;
  return 0;
}
int qmm_synchronize(qmm_stream s) {
  hipError_t e = hipStreamSynchronize(stream_of(s));
  if (e != hipSuccess) return finish(fail_hip(e, "qmm_synchronize"));
  return finish(0);
}

// ---------------- errors
int qmm_set_error_handler(qmm_error_handler_func handler, void *data, void (*dtor)(void *)) {
  std::lock_guard<std::mutex> lk(g_err_mtx);
  if (g_handler_dtor && g_handler_data) g_handler_dtor(g_handler_data);
  g_handler = handler;
  g_handler_data = data;
  g_handler_dtor = dtor;
  return 0;
}

bool qmm_error_pending(void) { return g_latched.load(std::memory_order_acquire); }

bool qmm_error_is_memory(const char *msg) {
  static const char *needles[] = {"Insufficient Memory", "insufficient memory", "Unable to allocate",
                                  "Resource limit",      "out of memory",       "Out of memory",
                                  "maximum allowed buffer size", "hipErrorOutOfMemory"};
  for (const char *n : needles)
    if (std::strstr(msg, n)) return true;
  return false;
}

const char *qmm_peek_error_name(void) {
  if (!g_latched.load(std::memory_order_acquire)) return nullptr;
  std::lock_guard<std::mutex> lk(g_err_mtx);
  return qmm_error_is_memory(g_err_buf) ? "OutOfMemory" : "MlxFailure";
}

int qmm_take_error(char *buf, size_t len) {
  if (!g_latched.load(std::memory_order_acquire)) return -1;
  std::lock_guard<std::mutex> lk(g_err_mtx);
  size_t n = g_err_len;
  if (buf && len) {
    size_t c = n < len - 1 ? n : len - 1;
    std::memcpy(buf, g_err_buf, c);
    buf[c] = 0;
  }
  g_err_len = 0;
  g_err_buf[0] = 0;
  g_latched.store(false, std::memory_order_release);
  return (int)n;
}

static int consume_latch() {
  if (!g_latched.load(std::memory_order_acquire)) return 0;
  char buf[512];
  if (qmm_take_error(buf, sizeof buf) < 0) return 0;
  return qmm_error_is_memory(buf) ? QMM_ERR_OOM : QMM_ERR_FAILURE;
}

// An error the HIP runtime holds for the calling thread (a failed call, or a launch or
// device error a synchronising call reported) joins the latch first.  Nothing here
// waits for the device: errors of work still in flight surface at the call that waits
// for it (qmm_synchronize, qmm_array_to_host), which latches them.
// Without a device the runtime answers every call with hipErrorNoDevice: that is no
// work's error (an op that needs the device reports it itself).  hipErrorNotReady is the
// answer of a query (hipStreamQuery, hipEventQuery) whose work has not finished yet, which
// the caller's own polling leaves behind: a status, not a failure.
static void latch_runtime_error() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess && e != hipErrorNoDevice && e != hipErrorNotReady)
    fail_hip(e, "qmm_check_error: pending HIP runtime error");
}
int qmm_check_error(void) {
  latch_runtime_error();
  g_fault_chunk.maybe_fire();
  return consume_latch();
}
int qmm_check_error_decode(void) {
  latch_runtime_error();
  g_fault_step.maybe_fire();
  return consume_latch();
}
void qmm_latch_error_for_test(const char *msg) { latch_error(msg); }
void qmm_reset_faults_for_test(void) {
  g_fault_chunk.reset();
  g_fault_step.reset();
  qmm_take_error(nullptr, 0);
}
void qmm_fault_arm(uint64_t k) {
  g_fault_remaining = k;
  g_fault_fired = false;
}
bool qmm_fault_did_fire(void) { return g_fault_fired; }
uint64_t qmm_op_count(void) { return g_op_count.load(std::memory_order_relaxed); }

// ---------------- vector_array
qmm_vector_array qmm_vector_array_new(void) { return qmm_vector_array{new VecArr()}; }
int qmm_vector_array_free(qmm_vector_array v) {
  VecArr *p = (VecArr *)v.ctx;
  if (!p) return 0;
  for (Arr *a : p->items) release_arr(a);
  delete p;
  return 0;
}
size_t qmm_vector_array_size(qmm_vector_array v) { return v.ctx ? ((VecArr *)v.ctx)->items.size() : 0; }
int qmm_vector_array_get(qmm_array *res, qmm_vector_array v, size_t idx) {
  VecArr *p = (VecArr *)v.ctx;
  if (!p || idx >= p->items.size()) return finish(fail("[qmm_vector_array_get] index %zu out of range", idx));
  // A new borrowed view of the vector's array (the vector keeps ownership, as
  // mlx arrays share their buffer); free the view with qmm_array_free.
  Arr *src = p->items[idx];
  Arr *a = new_arr(src->shape, src->ndim, src->dtype);
  a->data = src->data;
  a->owned = false;
  if (res->ctx) release_arr((Arr *)res->ctx);
  res->ctx = a;
  return finish(0);
}

// ---------------- ops
static int parse_mode(const char *mode, qmm_optional_int gs, qmm_optional_int bits, const char *op, int *m_out) {
  if (!mode) return fail("[%s] mode is null", op);
  int m;
  if (std::strcmp(mode, "mxfp8") == 0)
    m = MXFP8;
  else if (std::strcmp(mode, "nvfp4") == 0)
    m = NVFP4;
  else
    return fail("[%s] Unsupported quantization mode '%s' (this library serves mxfp8 and nvfp4)", op, mode);
  const int g = m == MXFP8 ? 32 : 16, b = m == MXFP8 ? 8 : 4;
  if (gs.has_value && gs.value != g) return fail("[%s] %s requires group_size %d, got %d", op, mode, g, gs.value);
  if (bits.has_value && bits.value != b) return fail("[%s] %s requires bits %d, got %d", op, mode, b, bits.value);
  *m_out = m;
  return 0;
}

// Validate packed weights + scales, derive N and K.
static int check_wq(const Arr *w, const Arr *sc, int mode, const char *op, int *N, int *K) {
  const int g = mode == MXFP8 ? 32 : 16, bits = mode == MXFP8 ? 8 : 4;
  if (!w || !sc) return fail("[%s] missing weight or scales", op);
  if (w->dtype != QMM_UINT32 || w->ndim != 2)
    return fail("[%s] packed weight must be a 2D uint32 array", op);
  if (sc->dtype != QMM_UINT8 || sc->ndim != 2) return fail("[%s] scales must be a 2D uint8 array", op);
  *N = w->shape[0];
  *K = (int)((int64_t)w->shape[1] * 32 / bits);
  if (sc->shape[0] != *N || (int64_t)sc->shape[1] * g != *K)
    return fail("[%s] scales shape [%d, %d] does not match weight [%d, %d] for group %d", op, sc->shape[0],
                sc->shape[1], w->shape[0], w->shape[1], g);
  return 0;
}

// The scales of `sa` in the prefill GEMMs' tile-major layout, made once per handle and kept
// with it: mlx arrays are immutable, so the contents behind a handle do not change while it
// lives.  *out is null when the GEMM for `a` reads the scales as stored, while the stream is
// being captured and no copy exists yet (it would become part of the graph), or if the copy
// cannot be allocated; the GEMM then repacks into its workspace on every call.
//
// The copy is published only once it is complete on the device: a plain allocation (not
// stream-ordered), the repack on the caller's stream, then a wait for that stream.  A call
// on any other stream or thread that finds the pointer can read it with no further
// ordering, and freeing it (release_tiled) does not need the stream that made it.  The
// wait happens once per handle, at its first prefill call.  Returns non-zero, with the
// error latched, only when the stream reports a device error.
static std::mutex g_tiled_mtx;
static int tiled_scales(Arr *sa, const QmmArgs &a, hipStream_t st, const uint32_t **out) {
  *out = nullptr;
  const int nb = gemm_tiled_scale_bytes_per_row(a);
  if (!nb || !sa || sa->ndim != 2 || sa->shape[0] != a.N || sa->shape[1] != nb) return 0;
  std::lock_guard<std::mutex> lk(g_tiled_mtx);
  if (sa->tiled) {  // nb is the handle's own row length, so an existing copy always fits
    *out = (const uint32_t *)sa->tiled;
    return 0;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return 0;
  }
  const size_t bytes = tiled_scales_bytes(a.N, nb);
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  hipError_t e = launch_repack_scales(a.s, (int64_t)a.N, nb, (uint32_t *)p, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return fail_hip(e, "qmm::tiled_scales");
  }
  sa->tiled = p;
  sa->tiled_bytes = bytes;
  g_tiled_bytes.fetch_add(bytes, std::memory_order_relaxed);
  *out = (const uint32_t *)p;
  return 0;
}

// Whether a grouped call's stacked matrices can run as one prefill GEMM: the pipelined
// kernels (mxfp8: K % 128, scales 4-byte aligned), whose epilogues store to parts.
static bool gemm_parts_ok(const QmmArgs &a) {
  if (a.x_f32 || (((uintptr_t)a.x | (uintptr_t)a.w) & 15) != 0) return false;
  if (a.mode == MXFP8) return gemm_mxfp8_ok(a) && a.K % 128 == 0 && ((uintptr_t)a.s & 3) == 0;
  return gemm_nvfp4_ok(a);
}

// Workspace bytes run_qmm needs for these arguments (0 for the decode kernels).
static size_t qmm_workspace(const QmmArgs &a) {
  if (qmm_on_decode(a) || a.K == 0 || (((uintptr_t)a.x | (uintptr_t)a.w) & 15) != 0) return 0;
  if (gemm_mxfp8_ok(a)) return gemm_mxfp8_workspace(a);
  if (gemm_nvfp4_ok(a)) return gemm_nvfp4_workspace(a);
  return 0;
}

// y = x @ deq(W).T for the prepared arguments: picks the kernel family by shape.  The
// prefill GEMMs take their workspace from ws_given (qmm_workspace(a) bytes) or else the
// stream's.  Returns 0, or non-zero with the error latched.
static int run_qmm(QmmArgs &a, size_t ybytes, hipStream_t st, const char *op, void *ws_given = nullptr,
                   Arr *scales_arr = nullptr) {
  const int K = a.K, N = a.N;
  const bool aligned = (((uintptr_t)a.x | (uintptr_t)a.w) & 15) == 0;
  hipError_t e = hipSuccess;
  if (K == 0) {
    e = launch_fill_zero(a.y, ybytes, st);
  } else if (qmm_on_decode(a)) {
    if (qmv_mfma_ok(a))
      e = launch_qmv_mfma(a, st);
    else
      e = (aligned && qmv_fast_ok(a)) ? launch_qmv(a, st) : launch_qmv_generic(a, st);
  } else if (aligned && (gemm_mxfp8_ok(a) || gemm_nvfp4_ok(a))) {
    const bool fp8 = gemm_mxfp8_ok(a);
    if (!a.s_tiled && tiled_scales(scales_arr, a, st, &a.s_tiled)) return 1;
    const size_t need = fp8 ? gemm_mxfp8_workspace(a) : gemm_nvfp4_workspace(a);
    void *ws = ws_given;
    bool transient = false;
    if (!ws && workspace(st, need, &ws, &transient)) return 1;
    e = fp8 ? launch_gemm_mxfp8(a, ws, st) : launch_gemm_nvfp4(a, ws, st);
    if (transient) (void)hipFreeAsync(ws, st);  // stream-ordered: released after the kernels that use it
  } else if (aligned && gemm_ok(a)) {
    e = launch_gemm(a, st);
  } else {
    // f32 x (or an unaligned view) with many rows: decode kernel over row blocks of 8.
    const size_t esz = a.x_f32 ? 4 : 2;
    for (int m0 = 0; m0 < a.M && e == hipSuccess; m0 += QMV_MAX_M) {
      QmmArgs b = a;
      b.M = a.M - m0 < QMV_MAX_M ? a.M - m0 : QMV_MAX_M;
      b.x = (const char *)a.x + (size_t)m0 * K * esz;
      b.y = (char *)a.y + (size_t)m0 * N * esz;
      const bool al = (((uintptr_t)b.x | (uintptr_t)b.w) & 15) == 0;
      e = (al && qmv_fast_ok(b)) ? launch_qmv(b, st) : launch_qmv_generic(b, st);
    }
  }
  if (e != hipSuccess) return fail_hip(e, op);
  return 0;
}

int qmm_quantized_matmul(qmm_array *res, qmm_array x, qmm_array w, qmm_array scales, qmm_array biases,
                         bool transpose_w, qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                         qmm_stream s) {
  begin_op();
  const char *op = "quantized_matmul";
  if (!res) return finish(fail("[%s] null result pointer", op));
  int m;
  if (parse_mode(mode, group_size, bits, op, &m)) return finish(1);
  if (biases.ctx) return finish(fail("[%s] %s takes no biases", op, mode));
  if (!transpose_w) return finish(fail("[%s] only transpose_w = true is supported", op));
  Arr *xa = (Arr *)x.ctx, *wa = (Arr *)w.ctx, *sa = (Arr *)scales.ctx;
  if (!xa) return finish(fail("[%s] missing x", op));
  int N, K;
  if (check_wq(wa, sa, m, op, &N, &K)) return finish(1);
  if (xa->dtype != QMM_BFLOAT16 && xa->dtype != QMM_FLOAT32)
    return finish(fail("[%s] x must be bfloat16 or float32", op));
  if (xa->ndim < 1) return finish(fail("[%s] x must have at least one dimension", op));
  if (xa->shape[xa->ndim - 1] != K)
    return finish(fail("[%s] Last dimension of x (%d) does not match the weight's K (%d)", op,
                       xa->shape[xa->ndim - 1], K));
  int64_t M = 1;
  for (int i = 0; i < xa->ndim - 1; ++i) M *= xa->shape[i];
  if (M > INT32_MAX) return finish(fail("[%s] too many rows", op));
  std::vector<int> oshape(xa->shape, xa->shape + xa->ndim);
  oshape.back() = N;
  hipStream_t st = stream_of(s);
  Arr *ya;
  if (alloc_arr(res, oshape, xa->dtype, st, &ya)) return finish(1);
  if (M == 0 || N == 0) return finish(0);

  QmmArgs a;
  a.mode = m;
  a.x_f32 = xa->dtype == QMM_FLOAT32;
  a.M = (int)M;
  a.N = N;
  a.K = K;
  a.x = xa->data;
  a.w = (const uint8_t *)wa->data;
  a.s = (const uint8_t *)sa->data;
  a.y = ya->data;
  if (run_qmm(a, ya->nbytes(), st, op, nullptr, sa)) return finish(1);
  return finish(0);
}

// n projections of one x (the GDN layer's in_proj_qkv / z / b / a, src/model.zig:
// 1066-1074; attention's q / k / v, :929-944).  When the matrices, and their
// scales, lie back to back in memory (in any order) and the shape is a decode
// shape, one kernel runs over them as one matrix and writes each part's rows to
// its own result.
static std::atomic<uint64_t> g_group_launches{0};
uint64_t qmm_group_launch_count(void) { return g_group_launches.load(std::memory_order_relaxed); }
uint64_t qmm_scale_copy_bytes(void) { return g_tiled_bytes.load(std::memory_order_relaxed); }

int qmm_quantized_matmul_group(qmm_array *res, size_t n, qmm_array x, const qmm_array *w, const qmm_array *scales,
                               qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                               qmm_stream s) {
  begin_op();
  const char *op = "quantized_matmul_group";
  if (!res || !w || !scales) return finish(fail("[%s] null argument", op));
  if (n < 1 || n > 4) return finish(fail("[%s] takes 1 to 4 matrices, got %zu", op, n));
  int m;
  if (parse_mode(mode, group_size, bits, op, &m)) return finish(1);
  Arr *xa = (Arr *)x.ctx;
  if (!xa) return finish(fail("[%s] missing x", op));
  if (xa->dtype != QMM_BFLOAT16 && xa->dtype != QMM_FLOAT32)
    return finish(fail("[%s] x must be bfloat16 or float32", op));
  if (xa->ndim < 1) return finish(fail("[%s] x must have at least one dimension", op));
  int N[4], K = 0;
  for (size_t i = 0; i < n; ++i) {
    int Ki;
    if (check_wq((Arr *)w[i].ctx, (Arr *)scales[i].ctx, m, op, &N[i], &Ki)) return finish(1);
    if (i > 0 && Ki != K) return finish(fail("[%s] matrix %zu has K = %d, matrix 0 has %d", op, i, Ki, K));
    K = Ki;
  }
  if (xa->shape[xa->ndim - 1] != K)
    return finish(fail("[%s] Last dimension of x (%d) does not match the weights' K (%d)", op,
                       xa->shape[xa->ndim - 1], K));
  int64_t M = 1;
  for (int i = 0; i < xa->ndim - 1; ++i) M *= xa->shape[i];
  if (M > INT32_MAX) return finish(fail("[%s] too many rows", op));
  hipStream_t st = stream_of(s);
  Arr *ya[4];
  for (size_t i = 0; i < n; ++i) {
    std::vector<int> oshape(xa->shape, xa->shape + xa->ndim);
    oshape.back() = N[i];
    if (alloc_arr(&res[i], oshape, xa->dtype, st, &ya[i])) return finish(1);
  }
  if (M == 0) return finish(0);
  QmmArgs a;
  a.mode = m;
  a.x_f32 = xa->dtype == QMM_FLOAT32;
  a.M = (int)M;
  a.K = K;
  a.x = xa->data;
  // back to back: sorted by address, each matrix starts where the previous one ends
  int ord[4] = {0, 1, 2, 3};
  std::sort(ord, ord + n, [&](int i, int j) { return ((Arr *)w[i].ctx)->data < ((Arr *)w[j].ctx)->data; });
  const int64_t wrow = m == MXFP8 ? K : K / 2, srow = K / (m == MXFP8 ? 32 : 16);
  const uint8_t *w0 = (const uint8_t *)((Arr *)w[ord[0]].ctx)->data;
  const uint8_t *s0 = (const uint8_t *)((Arr *)scales[ord[0]].ctx)->data;
  bool together = K > 0;
  int64_t rows = 0;
  QmmParts parts;
  parts.n = (int)n;
  for (size_t j = 0; j < n; ++j) {
    const int i = ord[j];
    together = together && N[i] > 0 && (const uint8_t *)((Arr *)w[i].ctx)->data == w0 + rows * wrow &&
               (const uint8_t *)((Arr *)scales[i].ctx)->data == s0 + rows * srow;
    parts.y[j] = ya[i]->data;
    parts.rows[j] = N[i];
    rows += N[i];
  }
  if (together && rows <= INT32_MAX) {
    a.N = (int)rows;
    a.w = w0;
    a.s = s0;
    a.y = nullptr;
    a.parts = &parts;
    if (qmv_parts_ok(a)) {
      const hipError_t e = qmv_mfma_ok(a) ? launch_qmv_mfma(a, st) : launch_qmv(a, st);
      if (e != hipSuccess) return finish(fail_hip(e, op));
      g_group_launches.fetch_add(1, std::memory_order_relaxed);
      return finish(0);
    }
    // prefill shapes: one GEMM over the stacked matrices (one x split, one tiling of all
    // their rows, so narrow members share rounds with the wide ones), each output column
    // stored to its part.  The scales are repacked per call (no handle holds the stack's).
    if (!qmm_on_decode(a) && gemm_parts_ok(a)) {
      if (run_qmm(a, 0, st, op)) return finish(1);
      g_group_launches.fetch_add(1, std::memory_order_relaxed);
      return finish(0);
    }
  }
  // otherwise one call per matrix
  for (size_t i = 0; i < n; ++i) {
    if (N[i] == 0) continue;
    QmmArgs b;
    b.mode = m;
    b.x_f32 = a.x_f32;
    b.M = (int)M;
    b.N = N[i];
    b.K = K;
    b.x = xa->data;
    b.w = (const uint8_t *)((Arr *)w[i].ctx)->data;
    b.s = (const uint8_t *)((Arr *)scales[i].ctx)->data;
    b.y = ya[i]->data;
    if (run_qmm(b, ya[i]->nbytes(), st, op, nullptr, (Arr *)scales[i].ctx)) return finish(1);
  }
  return finish(0);
}

int qmm_silu_mul(qmm_array *res, qmm_array g, qmm_array u, qmm_stream s) {
  begin_op();
  const char *op = "silu_mul";
  if (!res) return finish(fail("[%s] null result pointer", op));
  Arr *ga = (Arr *)g.ctx, *ua = (Arr *)u.ctx;
  if (!ga || !ua) return finish(fail("[%s] missing input", op));
  if (ga->dtype != ua->dtype || (ga->dtype != QMM_BFLOAT16 && ga->dtype != QMM_FLOAT32))
    return finish(fail("[%s] inputs must both be bfloat16 or both float32", op));
  if (ga->ndim != ua->ndim) return finish(fail("[%s] shapes differ", op));
  for (int i = 0; i < ga->ndim; ++i)
    if (ga->shape[i] != ua->shape[i]) return finish(fail("[%s] shapes differ", op));
  std::vector<int> shape(ga->shape, ga->shape + ga->ndim);
  hipStream_t st = stream_of(s);
  Arr *ha;
  if (alloc_arr(res, shape, ga->dtype, st, &ha)) return finish(1);
  const int64_t n = (int64_t)ga->size();
  hipError_t e = launch_silu_mul(ga->data, ua->data, ha->data, n, ga->dtype == QMM_FLOAT32, st);
  if (e != hipSuccess) return finish(fail_hip(e, op));
  return finish(0);
}

// Validates the arguments of the GDN recurrence (shapes and dtypes of gdnKernelRun's
// inputs, src/model.zig:284-319, and fusedEligible, :322-329) into *a, all but the
// output pointers.  Returns 0, or non-zero with the error latched.
static int gdn_args(const char *op, qmm_array q, qmm_array k, qmm_array v, qmm_array g, qmm_array beta,
                    qmm_array state, qmm_dtype y_dtype, GdnArgs *a) {
  Arr *qa = (Arr *)q.ctx, *ka = (Arr *)k.ctx, *va = (Arr *)v.ctx, *ga = (Arr *)g.ctx, *ba = (Arr *)beta.ctx,
      *sa = (Arr *)state.ctx;
  if (!qa || !ka || !va || !ga || !ba || !sa) return fail("[%s] missing input", op);
  if (qa->ndim != 4 || ka->ndim != 4 || va->ndim != 4 || sa->ndim != 4)
    return fail("[%s] q, k, v and state must be 4-D", op);
  const int B = qa->shape[0], T = qa->shape[1], Hk = qa->shape[2], Dk = qa->shape[3];
  const int Hv = va->shape[2], Dv = va->shape[3];
  for (int i = 0; i < 4; ++i)
    if (ka->shape[i] != qa->shape[i]) return fail("[%s] q and k shapes differ", op);
  if (va->shape[0] != B || va->shape[1] != T) return fail("[%s] v must be [B, T, Hv, Dv]", op);
  if (ga->ndim != 3 || ga->shape[0] != B || ga->shape[1] != T || ga->shape[2] != Hv)
    return fail("[%s] g must be [B, T, Hv]", op);
  if (ba->ndim != 3 || ba->shape[0] != B || ba->shape[1] != T || ba->shape[2] != Hv)
    return fail("[%s] beta must be [B, T, Hv]", op);
  if (sa->shape[0] != B || sa->shape[1] != Hv || sa->shape[2] != Dv || sa->shape[3] != Dk)
    return fail("[%s] state must be [B, Hv, Dv, Dk]", op);
  if (qa->dtype != ka->dtype || qa->dtype != va->dtype || (qa->dtype != QMM_BFLOAT16 && qa->dtype != QMM_FLOAT32))
    return fail("[%s] q, k, v must all be bfloat16 or all float32", op);
  if (ga->dtype != QMM_FLOAT32 || sa->dtype != QMM_FLOAT32) return fail("[%s] g and state must be float32", op);
  if (ba->dtype != QMM_BFLOAT16 && ba->dtype != QMM_FLOAT32) return fail("[%s] beta must be bfloat16 or float32", op);
  if (y_dtype != QMM_BFLOAT16 && y_dtype != QMM_FLOAT32) return fail("[%s] y must be bfloat16 or float32", op);
  if (Dk != 128 || Dv <= 0 || Dv % 8 != 0 || Hk <= 0 || Hv % Hk != 0)
    return fail("[%s] needs Dk = 128, Dv a multiple of 8 and Hv a multiple of Hk (got Dk %d, Dv %d, Hk %d, Hv %d)",
                op, Dk, Dv, Hk, Hv);
  if ((((uintptr_t)qa->data) | ((uintptr_t)ka->data) | ((uintptr_t)sa->data)) & 15)
    return fail("[%s] q, k and state must be 16-byte aligned", op);
  a->B = B, a->T = T, a->Hk = Hk, a->Hv = Hv, a->Dk = Dk, a->Dv = Dv;
  a->in_f32 = qa->dtype == QMM_FLOAT32;
  a->beta_f32 = ba->dtype == QMM_FLOAT32;
  a->y_f32 = y_dtype == QMM_FLOAT32;
  a->q = qa->data, a->k = ka->data, a->v = va->data, a->beta = ba->data;
  a->g = (const float *)ga->data, a->state_in = (const float *)sa->data;
  a->state_out = nullptr, a->y = nullptr;
  return 0;
}

// T = 0: no steps, the state passes through (a copy unless the update is in place).
static hipError_t gdn_no_steps(const GdnArgs &a, hipStream_t st) {
  if (a.state_out == a.state_in) return hipSuccess;
  const size_t bytes = (size_t)a.B * a.Hv * a.Dv * a.Dk * sizeof(float);
  return hipMemcpyAsync(a.state_out, a.state_in, bytes, hipMemcpyDeviceToDevice, st);
}

int qmm_gdn_recurrence(qmm_array *y, qmm_array *state_out, qmm_array q, qmm_array k, qmm_array v, qmm_array g,
                       qmm_array beta, qmm_array state, qmm_dtype y_dtype, qmm_stream s) {
  begin_op();
  const char *op = "gdn_recurrence";
  if (!y || !state_out) return finish(fail("[%s] null result pointer", op));
  GdnArgs a;
  if (gdn_args(op, q, k, v, g, beta, state, y_dtype, &a)) return finish(1);
  hipStream_t st = stream_of(s);
  Arr *ya, *so;
  if (alloc_arr(y, {a.B, a.T, a.Hv, a.Dv}, y_dtype, st, &ya)) return finish(1);
  if (alloc_arr(state_out, {a.B, a.Hv, a.Dv, a.Dk}, QMM_FLOAT32, st, &so)) return finish(1);
  if (((uintptr_t)so->data) & 15) return finish(fail("[%s] state_out must be 16-byte aligned", op));
  a.state_out = (float *)so->data, a.y = ya->data;
  if ((int64_t)a.B * a.Hv == 0) return finish(0);
  hipError_t e;
  if (a.T == 0) {
    e = gdn_no_steps(a, st);
  } else if (gdn_chunked_ok(a)) {  // long T: the chunked form, its per-chunk matrices in the stream's workspace
    void *ws = nullptr;
    bool transient = false;
    if (workspace(st, gdn_chunked_workspace(a), &ws, &transient)) return finish(1);
    e = launch_gdn_chunked(a, ws, st);
    if (transient) (void)hipFreeAsync(ws, st);  // stream-ordered: released after the kernels that use it
  } else {
    e = launch_gdn(a, st);
  }
  if (e != hipSuccess) return finish(fail_hip(e, op));
  return finish(0);
}

// The result array *res must already hold exactly this shape and dtype.
static int preallocated(const char *op, const char *what, qmm_array *res, const std::vector<int> &shape,
                        qmm_dtype dtype, Arr **out) {
  Arr *a = res ? (Arr *)res->ctx : nullptr;
  bool same = a && a->data && a->dtype == dtype && a->ndim == (int)shape.size();
  for (int i = 0; same && i < a->ndim; ++i) same = a->shape[i] == shape[i];
  if (!same)
    return fail("[%s] %s must already hold an array of the result's shape and dtype: this entry point allocates "
                "nothing", op, what);
  *out = a;
  return 0;
}

int qmm_gdn_recurrence_noalloc(qmm_array *y, qmm_array *state_out, qmm_array q, qmm_array k, qmm_array v,
                               qmm_array g, qmm_array beta, qmm_array state, qmm_dtype y_dtype, qmm_stream s) {
  begin_op();
  const char *op = "gdn_recurrence_noalloc";
  if (!y || !state_out) return finish(fail("[%s] null result pointer", op));
  GdnArgs a;
  if (gdn_args(op, q, k, v, g, beta, state, y_dtype, &a)) return finish(1);
  Arr *ya, *so;
  if (preallocated(op, "*y", y, {a.B, a.T, a.Hv, a.Dv}, y_dtype, &ya)) return finish(1);
  if (preallocated(op, "*state_out", state_out, {a.B, a.Hv, a.Dv, a.Dk}, QMM_FLOAT32, &so)) return finish(1);
  if (((uintptr_t)so->data) & 15) return finish(fail("[%s] state_out must be 16-byte aligned", op));
  a.state_out = (float *)so->data, a.y = ya->data;
  hipStream_t st = stream_of(s);
  if ((int64_t)a.B * a.Hv == 0) return finish(0);
  hipError_t e;
  if (a.T == 0) {
    e = gdn_no_steps(a, st);
  } else if (gdn_chunked_ok(a)) {  // the chunked form, its workspace in the library's static array
    if (!gdn_noalloc_fits(a)) {
      GdnArgs one = a;  // one batch, one chunk: the least a launch needs
      one.B = 1, one.T = 1;
      return finish(fail("[%s] %d value heads need %zu bytes of workspace per 64-step chunk; the static workspace "
                         "holds %zu bytes",
                         op, a.Hv, gdn_chunked_workspace(one), gdn_noalloc_scratch_bytes()));
    }
    e = launch_gdn_chunked_noalloc(a, st);
  } else {
    e = launch_gdn(a, st);
  }
  if (e != hipSuccess) return finish(fail_hip(e, op));
  return finish(0);
}

int qmm_mlp_gate_up_silu(qmm_array *res, qmm_array x, qmm_array w_gate, qmm_array s_gate, qmm_array w_up,
                         qmm_array s_up, qmm_optional_int group_size, qmm_optional_int bits, const char *mode,
                         qmm_stream s) {
  begin_op();
  const char *op = "mlp_gate_up_silu";
  if (!res) return finish(fail("[%s] null result pointer", op));
  int m;
  if (parse_mode(mode, group_size, bits, op, &m)) return finish(1);
  Arr *xa = (Arr *)x.ctx;
  if (!xa) return finish(fail("[%s] missing x", op));
  int N, K, N2, K2;
  if (check_wq((Arr *)w_gate.ctx, (Arr *)s_gate.ctx, m, op, &N, &K)) return finish(1);
  if (check_wq((Arr *)w_up.ctx, (Arr *)s_up.ctx, m, op, &N2, &K2)) return finish(1);
  if (N != N2 || K != K2) return finish(fail("[%s] gate [%d, %d] and up [%d, %d] differ", op, N, K, N2, K2));
  if (xa->dtype != QMM_BFLOAT16 && xa->dtype != QMM_FLOAT32)
    return finish(fail("[%s] x must be bfloat16 or float32", op));
  if (xa->ndim < 1 || xa->shape[xa->ndim - 1] != K)
    return finish(fail("[%s] Last dimension of x does not match the weight's K (%d)", op, K));
  int64_t M = 1;
  for (int i = 0; i < xa->ndim - 1; ++i) M *= xa->shape[i];
  if (M > INT32_MAX) return finish(fail("[%s] too many rows", op));
  std::vector<int> oshape(xa->shape, xa->shape + xa->ndim);
  oshape.back() = N;
  hipStream_t st = stream_of(s);
  Arr *ha;
  if (alloc_arr(res, oshape, xa->dtype, st, &ha)) return finish(1);
  if (M == 0 || N == 0) return finish(0);
  QmmArgs a;
  a.mode = m;
  a.x_f32 = xa->dtype == QMM_FLOAT32;
  a.M = (int)M;
  a.N = N;
  a.K = K;
  a.x = xa->data;
  a.w = (const uint8_t *)((Arr *)w_gate.ctx)->data;
  a.s = (const uint8_t *)((Arr *)s_gate.ctx)->data;
  a.y = ha->data;
  const uint8_t *wu = (const uint8_t *)((Arr *)w_up.ctx)->data, *su = (const uint8_t *)((Arr *)s_up.ctx)->data;
  // decode shapes: one kernel for both projections and the activation.  Each
  // fused kernel computes the same per-row sums as the kernel run_qmm picks
  // for the shape, so the fused result equals the unfused one.
  if (K > 0 && qmv_mfma_ok(a)) {
    if (qmv_mfma_mlp_ok(a, wu, su)) {
      hipError_t e = launch_qmv_mfma_mlp(a, wu, su, st);
      if (e != hipSuccess) return finish(fail_hip(e, op));
      return finish(0);
    }
  } else if (K > 0 && qmv_mlp_ok(a) && ((uintptr_t)wu & 15) == 0) {
    hipError_t e = launch_qmv_mlp(a, wu, su, st);
    if (e != hipSuccess) return finish(fail_hip(e, op));
    return finish(0);
  }
  // prefill shapes: the two projections, then the activation; the gate and up results
  // and the projections' own workspace in the stream's workspace
  const size_t bytes = (ha->nbytes() + 255) & ~(size_t)255;
  QmmArgs b = a;
  b.w = wu;
  b.s = su;
  if (tiled_scales((Arr *)s_gate.ctx, a, st, &a.s_tiled) || tiled_scales((Arr *)s_up.ctx, b, st, &b.s_tiled))
    return finish(1);
  const size_t gemm_ws = std::max(qmm_workspace(a), qmm_workspace(b));
  void *ws = nullptr;
  bool transient = false;
  if (workspace(st, 2 * bytes + gemm_ws, &ws, &transient)) return finish(1);
  void *g = ws, *u = (char *)ws + bytes, *gws = gemm_ws ? (char *)ws + 2 * bytes : nullptr;
  a.y = g;
  b.y = u;
  // mxfp8: the up projection reuses the x split the gate projection made in the shared
  // workspace (same x, M, K and split layout; the two launches are stream-ordered)
  const bool aligned_x = (((uintptr_t)a.x | (uintptr_t)a.w | (uintptr_t)b.w) & 15) == 0;
  b.x_split_ready = gws && aligned_x && gemm_mxfp8_ok(a) && gemm_mxfp8_ok(b) &&
                    gemm_mxfp8_split_layout_of(a) == gemm_mxfp8_split_layout_of(b);
  int rc = run_qmm(a, bytes, st, op, gws);
  if (!rc) rc = run_qmm(b, bytes, st, op, gws);
  if (!rc) {
    hipError_t e = launch_silu_mul(g, u, ha->data, (int64_t)M * N, a.x_f32, st);
    if (e != hipSuccess) rc = fail_hip(e, op);
  }
  if (transient) (void)hipFreeAsync(ws, st);  // stream-ordered: released after the kernels that use it
  return finish(rc ? 1 : 0);
}

int qmm_dequantize(qmm_array *res, qmm_array w, qmm_array scales, qmm_array biases, qmm_optional_int group_size,
                   qmm_optional_int bits, const char *mode, qmm_array global_scale, qmm_optional_dtype dtype,
                   qmm_stream s) {
  begin_op();
  const char *op = "dequantize";
  if (!res) return finish(fail("[%s] null result pointer", op));
  int m;
  if (parse_mode(mode, group_size, bits, op, &m)) return finish(1);
  if (biases.ctx) return finish(fail("[%s] %s takes no biases", op, mode));
  if (global_scale.ctx) return finish(fail("[%s] global_scale is not supported", op));
  qmm_dtype dt = dtype.has_value ? dtype.value : QMM_BFLOAT16;
  if (dt != QMM_BFLOAT16 && dt != QMM_FLOAT32) return finish(fail("[%s] dtype must be bfloat16 or float32", op));
  Arr *wa = (Arr *)w.ctx, *sa = (Arr *)scales.ctx;
  int N, K;
  if (check_wq(wa, sa, m, op, &N, &K)) return finish(1);
  hipStream_t st = stream_of(s);
  Arr *o;
  if (alloc_arr(res, {N, K}, dt, st, &o)) return finish(1);
  hipError_t e = launch_dequant(m, (const uint8_t *)wa->data, (const uint8_t *)sa->data, N, K, o->data,
                                dt == QMM_FLOAT32, st);
  if (e != hipSuccess) return finish(fail_hip(e, op));
  return finish(0);
}

int qmm_quantize(qmm_vector_array *res, qmm_array w, qmm_optional_int group_size, qmm_optional_int bits,
                 const char *mode, qmm_array global_scale, qmm_stream s) {
  begin_op();
  const char *op = "quantize";
  if (!res) return finish(fail("[%s] null result pointer", op));
  int m;
  if (parse_mode(mode, group_size, bits, op, &m)) return finish(1);
  if (global_scale.ctx) return finish(fail("[%s] global_scale is not supported", op));
  Arr *wa = (Arr *)w.ctx;
  if (!wa || wa->ndim != 2 || (wa->dtype != QMM_BFLOAT16 && wa->dtype != QMM_FLOAT32))
    return finish(fail("[%s] w must be a 2D bfloat16 or float32 array", op));
  const int g = m == MXFP8 ? 32 : 16, b = m == MXFP8 ? 8 : 4;
  const int N = wa->shape[0], K = wa->shape[1];
  if (K % g != 0) return finish(fail("[%s] the last dimension (%d) must be divisible by the group size %d", op, K, g));
  hipStream_t st = stream_of(s);
  VecArr *v = new VecArr();
  Arr *q = new_arr(std::vector<int>{N, K * b / 32}.data(), 2, QMM_UINT32);
  Arr *sc = new_arr(std::vector<int>{N, K / g}.data(), 2, QMM_UINT8);
  v->items = {q, sc};
  for (Arr *a : v->items) {
    a->owned = true;
    a->alloc_stream = st;
    if (alloc_device(&a->data, a->nbytes(), st)) {
      qmm_vector_array_free(qmm_vector_array{v});
      return finish(1);
    }
  }
  hipError_t e = launch_quantize(m, wa->data, wa->dtype == QMM_FLOAT32, N, K, (uint32_t *)q->data,
                                 (uint8_t *)sc->data, st);
  if (e != hipSuccess) {
    qmm_vector_array_free(qmm_vector_array{v});
    return finish(fail_hip(e, op));
  }
  if (res->ctx) qmm_vector_array_free(*res);
  res->ctx = v;
  return finish(0);
}

int qmm_linear(qmm_array *res, qmm_array x, qmm_array w, qmm_stream s) {
  begin_op();
  const char *op = "linear";
  if (!res) return finish(fail("[%s] null result pointer", op));
  Arr *xa = (Arr *)x.ctx, *wa = (Arr *)w.ctx;
  if (!xa || !wa) return finish(fail("[%s] missing x or w", op));
  if (xa->dtype != QMM_BFLOAT16 || wa->dtype != QMM_BFLOAT16 || wa->ndim != 2 || xa->ndim < 1)
    return finish(fail("[%s] x [..., K] and w [N, K] must be bfloat16", op));
  const int N = wa->shape[0], K = wa->shape[1];
  if (xa->shape[xa->ndim - 1] != K)
    return finish(fail("[matmul] Last dimension of first input (%d) must match the weight (%d)",
                       xa->shape[xa->ndim - 1], K));
  if (K % 16 != 0 || (((uintptr_t)xa->data | (uintptr_t)wa->data) & 15) != 0)
    return finish(fail("[%s] K must be a multiple of 16 and operands 16-byte aligned", op));
  int64_t M = 1;
  for (int i = 0; i < xa->ndim - 1; ++i) M *= xa->shape[i];
  std::vector<int> oshape(xa->shape, xa->shape + xa->ndim);
  oshape.back() = N;
  hipStream_t st = stream_of(s);
  Arr *ya;
  if (alloc_arr(res, oshape, QMM_BFLOAT16, st, &ya)) return finish(1);
  if (M == 0 || N == 0) return finish(0);
  hipError_t e = launch_linear_bf16((const uint16_t *)xa->data, (const uint16_t *)wa->data, (uint16_t *)ya->data,
                                    (int)M, N, K, st);
  if (e != hipSuccess) return finish(fail_hip(e, op));
  return finish(0);
}

}  // extern "C"
