// Internal host-side types shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/qmm.h"

namespace qmm {

constexpr int QMM_MAX_DIM = 8;

size_t dtype_size(qmm_dtype d);

// The object behind a qmm_array handle: an HBM buffer plus shape and dtype.
struct Arr {
  void *data = nullptr;
  bool owned = false;                   // free the buffer with the handle
  hipStream_t alloc_stream = nullptr;   // stream the buffer was allocated on (stream-ordered free)
  int ndim = 0;
  int shape[QMM_MAX_DIM] = {0};
  qmm_dtype dtype = QMM_BOOL;
  // For a scales array: a copy in the prefill GEMMs' tile-major layout (tiled_bytes bytes,
  // a plain allocation), made at the first prefill call that reads it, complete on the
  // device before it is set, and freed with the handle (release_tiled).
  void *tiled = nullptr;
  size_t tiled_bytes = 0;
  size_t size() const;
  size_t nbytes() const { return size() * dtype_size(dtype); }
};

struct Stream {
  hipStream_t h = nullptr;
};

struct VecArr {
  std::vector<Arr *> items;
};

void latch_error(const char *msg);
int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int fail_hip(hipError_t e, const char *what);
int finish(int rc);
// Clears an error the HIP runtime holds for this thread from outside the library (at the
// start of every op that launches work).
void begin_op();
int alloc_device(void **p, size_t bytes, hipStream_t st);
// Scratch for work enqueued on `st` (at least `bytes`): the stream's grow-only
// workspace, or while the stream is being captured and that is too small, a
// transient allocation (*transient) the caller releases after its kernels.
int workspace(hipStream_t st, size_t bytes, void **out, bool *transient);
Arr *new_arr(const int *shape, int dim, qmm_dtype dtype);
int alloc_arr(qmm_array *res, const std::vector<int> &shape, qmm_dtype dtype, hipStream_t st, Arr **out);
void release_arr(Arr *a);
// Frees the handle's tile-major scale copy, if it has one (waits for the device first).
void release_tiled(Arr *a);
hipStream_t stream_of(qmm_stream s);

}  // namespace qmm
