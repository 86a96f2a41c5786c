"""ctypes binding of libqmm.so (the C ABI declared in include/qmm.h).

This is the Python-side stub of the boundary: the same calls mlx-runner's Zig
code makes through `extern "c"` declarations (src/mlx.zig:265, :274, :278),
used by the tests and the benchmark.  Device memory may come from torch
(borrowed through `Array.from_torch`); torch is only plumbing here.

Importing this module loads libqmm.so and raises if it is missing: there is no
fallback path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_bool, c_char_p, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libqmm.so"
HEADER = HERE.parent / "include" / "qmm.h"

if not LIB_PATH.exists():
    raise ImportError(f"{LIB_PATH} is not built; run `python mlx-runner_amd/build.py` (hipcc, gfx950)")


class qmm_array(ctypes.Structure):
    _fields_ = [("ctx", c_void_p)]


class qmm_stream(ctypes.Structure):
    _fields_ = [("ctx", c_void_p)]


class qmm_vector_array(ctypes.Structure):
    _fields_ = [("ctx", c_void_p)]


class qmm_weight_map(ctypes.Structure):
    _fields_ = [("ctx", c_void_p)]


class qmm_optional_int(ctypes.Structure):
    _fields_ = [("value", c_int), ("has_value", c_bool)]


class qmm_optional_dtype(ctypes.Structure):
    _fields_ = [("value", c_int), ("has_value", c_bool)]


class qmm_quant_spec(ctypes.Structure):
    _fields_ = [("mode", c_int), ("group_size", c_uint32), ("bits", c_uint32)]


UINT8, UINT16, UINT32, INT32, FLOAT16, FLOAT32, BFLOAT16 = 1, 2, 3, 7, 9, 10, 12
ERR_OOM, ERR_FAILURE = 1, 2
QUANT_NONE, QUANT_MXFP8, QUANT_NVFP4 = 0, 1, 2
WE = {101: "BadIndexJson", 102: "BadHeader", 103: "UnsupportedDtype", 104: "UnsupportedLayout",
      105: "MissingTensor", 106: "DuplicateTensor", 107: "NonstandardQuant", 108: "InconsistentQuant",
      109: "AffineUnsupported", 110: "IO", 111: "MissingWeight"}

# torch ships its own libamdhip64.so (soname libamdhip64.so.7).  If libqmm.so
# were loaded first, its NEEDED entry would pull /opt/rocm's copy and torch
# would later load a second HIP runtime, which then sees no device.  Loading
# torch first makes libqmm.so bind to the runtime already in the process.
try:
    import torch as _torch  # noqa: F401
except ImportError:  # pure C-ABI use without torch: /opt/rocm's runtime is the only one
    _torch = None

lib = ctypes.CDLL(str(LIB_PATH))

ERROR_HANDLER = ctypes.CFUNCTYPE(None, c_char_p, c_void_p)
_SIGS = {
    "qmm_version": (c_char_p, []),
    "qmm_device_info": (c_int, [c_char_p, c_size_t]),
    "qmm_array_new": (qmm_array, []),
    "qmm_array_new_data": (qmm_array, [c_void_p, POINTER(c_int), c_int, c_int]),
    "qmm_array_new_device": (qmm_array, [c_void_p, POINTER(c_int), c_int, c_int]),
    "qmm_array_free": (c_int, [qmm_array]),
    "qmm_array_ndim": (c_size_t, [qmm_array]),
    "qmm_array_shape": (POINTER(c_int), [qmm_array]),
    "qmm_array_dtype": (c_int, [qmm_array]),
    "qmm_array_size": (c_size_t, [qmm_array]),
    "qmm_array_nbytes": (c_size_t, [qmm_array]),
    "qmm_array_data_device": (c_void_p, [qmm_array]),
    "qmm_array_to_host": (c_int, [c_void_p, c_size_t, qmm_array, qmm_stream]),
    "qmm_default_gpu_stream_new": (qmm_stream, []),
    "qmm_stream_new_from_hip": (qmm_stream, [c_void_p]),
    "qmm_stream_free": (c_int, [qmm_stream]),
    "qmm_synchronize": (c_int, [qmm_stream]),
    "qmm_quantized_matmul": (c_int, [POINTER(qmm_array), qmm_array, qmm_array, qmm_array, qmm_array, c_bool,
                                     qmm_optional_int, qmm_optional_int, c_char_p, qmm_stream]),
    "qmm_dequantize": (c_int, [POINTER(qmm_array), qmm_array, qmm_array, qmm_array, qmm_optional_int,
                               qmm_optional_int, c_char_p, qmm_array, qmm_optional_dtype, qmm_stream]),
    "qmm_quantize": (c_int, [POINTER(qmm_vector_array), qmm_array, qmm_optional_int, qmm_optional_int, c_char_p,
                             qmm_array, qmm_stream]),
    "qmm_vector_array_new": (qmm_vector_array, []),
    "qmm_vector_array_free": (c_int, [qmm_vector_array]),
    "qmm_vector_array_size": (c_size_t, [qmm_vector_array]),
    "qmm_vector_array_get": (c_int, [POINTER(qmm_array), qmm_vector_array, c_size_t]),
    "qmm_set_error_handler": (c_int, [ERROR_HANDLER, c_void_p, c_void_p]),
    "qmm_error_pending": (c_bool, []),
    "qmm_error_is_memory": (c_bool, [c_char_p]),
    "qmm_peek_error_name": (c_char_p, []),
    "qmm_take_error": (c_int, [c_char_p, c_size_t]),
    "qmm_check_error": (c_int, []),
    "qmm_check_error_decode": (c_int, []),
    "qmm_latch_error_for_test": (None, [c_char_p]),
    "qmm_reset_faults_for_test": (None, []),
    "qmm_fault_arm": (None, [c_uint64]),
    "qmm_fault_did_fire": (c_bool, []),
    "qmm_op_count": (c_uint64, []),
    "qmm_group_launch_count": (c_uint64, []),
    "qmm_scale_copy_bytes": (c_uint64, []),
    "qmm_infer_quant_spec_json": (c_int, [c_char_p, c_size_t, POINTER(qmm_quant_spec), POINTER(c_size_t)]),
    "qmm_parse_header_json": (c_int, [c_char_p, c_size_t, POINTER(c_size_t)]),
    "qmm_sanitize_name": (c_int, [c_char_p, c_char_p, c_size_t]),
    "qmm_weights_load": (c_int, [POINTER(qmm_weight_map), c_char_p, qmm_stream]),
    "qmm_weights_free": (c_int, [qmm_weight_map]),
    "qmm_weights_get": (qmm_array, [qmm_weight_map, c_char_p]),
    "qmm_weights_count": (c_size_t, [qmm_weight_map]),
    "qmm_weights_quant": (qmm_quant_spec, [qmm_weight_map]),
    "qmm_named_linear_q": (c_int, [POINTER(qmm_array), qmm_weight_map, qmm_array, c_char_p, qmm_stream]),
    "qmm_linear": (c_int, [POINTER(qmm_array), qmm_array, qmm_array, qmm_stream]),
    "qmm_silu_mul": (c_int, [POINTER(qmm_array), qmm_array, qmm_array, qmm_stream]),
    "qmm_gdn_recurrence": (c_int, [POINTER(qmm_array), POINTER(qmm_array), qmm_array, qmm_array, qmm_array,
                                   qmm_array, qmm_array, qmm_array, c_int, qmm_stream]),
    "qmm_gdn_recurrence_noalloc": (c_int, [POINTER(qmm_array), POINTER(qmm_array), qmm_array, qmm_array, qmm_array,
                                           qmm_array, qmm_array, qmm_array, c_int, qmm_stream]),
    "qmm_mlp_gate_up_silu": (c_int, [POINTER(qmm_array), qmm_array, qmm_array, qmm_array, qmm_array, qmm_array,
                                     qmm_optional_int, qmm_optional_int, c_char_p, qmm_stream]),
    "qmm_mlp_forward_q": (c_int, [POINTER(qmm_array), qmm_weight_map, qmm_array, c_char_p, c_char_p, c_char_p,
                                  qmm_stream]),
    "qmm_quantized_matmul_group": (c_int, [POINTER(qmm_array), c_size_t, qmm_array, POINTER(qmm_array),
                                           POINTER(qmm_array), qmm_optional_int, qmm_optional_int, c_char_p,
                                           qmm_stream]),
    "qmm_named_linear_q_group": (c_int, [POINTER(qmm_array), c_size_t, qmm_weight_map, qmm_array,
                                         POINTER(c_char_p), qmm_stream]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


class QmmError(RuntimeError):
    """An op returned non-zero; carries the latched message."""


def opt_int(v=None) -> qmm_optional_int:
    return qmm_optional_int(0, False) if v is None else qmm_optional_int(int(v), True)


def take_error() -> str | None:
    buf = ctypes.create_string_buffer(512)
    n = lib.qmm_take_error(buf, 512)
    return None if n < 0 else buf.value.decode()


def check(rc: int, what: str = "qmm"):
    """The `check` chokepoint of the reference binding (src/mlx.zig:589-595)."""
    if rc != 0:
        msg = take_error()
        raise QmmError(f"{what} failed (rc={rc}): {msg}")


_TORCH_DTYPES = None


def _torch_dtype_map():
    global _TORCH_DTYPES
    if _TORCH_DTYPES is None:
        import torch

        _TORCH_DTYPES = {torch.uint8: UINT8, torch.int32: UINT32, torch.bfloat16: BFLOAT16,
                         torch.float32: FLOAT32, torch.uint32: UINT32}
    return _TORCH_DTYPES


class Stream:
    def __init__(self, hip_stream: int | None = None):
        self.h = lib.qmm_default_gpu_stream_new() if hip_stream is None else lib.qmm_stream_new_from_hip(hip_stream)

    @classmethod
    def torch_current(cls) -> "Stream":
        import torch

        return cls(torch.cuda.current_stream().cuda_stream)

    def sync(self):
        check(lib.qmm_synchronize(self.h), "synchronize")

    def __del__(self):
        try:
            lib.qmm_stream_free(self.h)
        except Exception:
            pass


class Array:
    """Owns a qmm_array handle (freed on deletion)."""

    def __init__(self, h: qmm_array | None = None, keepalive=None):
        self.h = h if h is not None else lib.qmm_array_new()
        self._keep = keepalive

    @classmethod
    def from_torch(cls, t, dtype: int | None = None) -> "Array":
        """Borrow a contiguous CUDA tensor's HBM (no copy)."""
        assert t.is_cuda and t.is_contiguous()
        dt = dtype if dtype is not None else _torch_dtype_map()[t.dtype]
        shape = (c_int * max(t.dim(), 1))(*t.shape)
        h = lib.qmm_array_new_device(c_void_p(t.data_ptr()), shape, t.dim(), dt)
        if not h.ctx:
            check(1, "array_new_device")
        return cls(h, keepalive=t)

    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: int) -> "Array":
        a = np.ascontiguousarray(a)
        shape = (c_int * max(a.ndim, 1))(*a.shape)
        h = lib.qmm_array_new_data(c_void_p(a.ctypes.data), shape, a.ndim, dtype)
        if not h.ctx:
            check(1, "array_new_data")
        return cls(h)

    @property
    def shape(self):
        n = lib.qmm_array_ndim(self.h)
        p = lib.qmm_array_shape(self.h)
        return tuple(p[i] for i in range(n))

    @property
    def dtype(self) -> int:
        return lib.qmm_array_dtype(self.h)

    @property
    def ptr(self) -> int:
        return lib.qmm_array_data_device(self.h) or 0

    def numpy(self, stream: Stream | None = None) -> np.ndarray:
        npdt = {UINT8: np.uint8, UINT32: np.uint32, FLOAT32: np.float32, BFLOAT16: np.uint16}[self.dtype]
        out = np.empty(self.shape, dtype=npdt)
        s = stream or Stream()
        check(lib.qmm_array_to_host(c_void_p(out.ctypes.data), out.nbytes, self.h, s.h), "array_to_host")
        return out

    def free(self):
        if self.h is not None and self.h.ctx:
            lib.qmm_array_free(self.h)
        self.h = qmm_array(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _stream(stream):
    return stream if stream is not None else Stream()


def quantized_matmul(x: Array, w: Array, scales: Array, mode: str, *, group_size=None, bits=None,
                     out: Array | None = None, transpose: bool = True, biases: Array | None = None,
                     stream: Stream | None = None) -> Array:
    res = out if out is not None else Array()
    s = _stream(stream)
    check(lib.qmm_quantized_matmul(byref(res.h), x.h, w.h, scales.h, biases.h if biases else qmm_array(None),
                                   transpose, opt_int(group_size), opt_int(bits), mode.encode(), s.h),
          "quantized_matmul")
    return res


def dequantize(w: Array, scales: Array, mode: str, *, dtype: int | None = None, group_size=None, bits=None,
               stream: Stream | None = None) -> Array:
    res = Array()
    s = _stream(stream)
    od = qmm_optional_dtype(0, False) if dtype is None else qmm_optional_dtype(dtype, True)
    check(lib.qmm_dequantize(byref(res.h), w.h, scales.h, qmm_array(None), opt_int(group_size), opt_int(bits),
                             mode.encode(), qmm_array(None), od, s.h), "dequantize")
    return res


class _VectorHolder:
    """Keeps a qmm_vector_array (and so its buffers) alive while views exist."""

    def __init__(self, v: qmm_vector_array):
        self.v = v

    def __del__(self):
        try:
            lib.qmm_vector_array_free(self.v)
        except Exception:
            pass


def quantize(w: Array, mode: str, *, group_size=None, bits=None, stream: Stream | None = None):
    """(packed uint32 [N, K*bits/32], scales uint8 [N, K/group]), both resident in HBM."""
    v = lib.qmm_vector_array_new()
    s = _stream(stream)
    rc = lib.qmm_quantize(byref(v), w.h, opt_int(group_size), opt_int(bits), mode.encode(), qmm_array(None), s.h)
    holder = _VectorHolder(v)
    check(rc, "quantize")
    outs = []
    for i in range(lib.qmm_vector_array_size(v)):
        view = Array(keepalive=holder)
        check(lib.qmm_vector_array_get(byref(view.h), v, i), "vector_array_get")
        outs.append(view)
    return outs[0], outs[1]


def linear(x: Array, w: Array, *, out: Array | None = None, stream: Stream | None = None) -> Array:
    res = out if out is not None else Array()
    s = _stream(stream)  # keep the wrapper alive across the call (its __del__ frees the handle)
    check(lib.qmm_linear(byref(res.h), x.h, w.h, s.h), "linear")
    return res


def silu_mul(g: Array, u: Array, *, out: Array | None = None, stream: Stream | None = None) -> Array:
    """silu(g) * u with the reference's per-op roundings (src/model.zig:405-415, :451-456)."""
    res = out if out is not None else Array()
    s = _stream(stream)
    check(lib.qmm_silu_mul(byref(res.h), g.h, u.h, s.h), "silu_mul")
    return res


def gdn_recurrence(q: Array, k: Array, v: Array, g: Array, beta: Array, state: Array, *, y_dtype: int = BFLOAT16,
                   y: Array | None = None, state_out: Array | None = None,
                   stream: Stream | None = None) -> tuple[Array, Array]:
    """The packed gated-delta recurrence (gdnKernelRun, src/model.zig:284-319):
    returns (y [B, T, Hv, Dv] in y_dtype, final state [B, Hv, Dv, Dk] float32).
    Pass state_out=state to update the state in place."""
    yr = y if y is not None else Array()
    so = state_out if state_out is not None else Array()
    s = _stream(stream)
    check(lib.qmm_gdn_recurrence(byref(yr.h), byref(so.h), q.h, k.h, v.h, g.h, beta.h, state.h, y_dtype, s.h),
          "gdn_recurrence")
    return yr, so


def gdn_recurrence_noalloc(q: Array, k: Array, v: Array, g: Array, beta: Array, state: Array, *, y: Array,
                           state_out: Array, y_dtype: int = BFLOAT16, stream: Stream | None = None):
    """qmm_gdn_recurrence_noalloc: the recurrence into caller-held results (y and
    state_out must already be arrays of the result shapes; state_out may be state),
    allocating nothing: the chunked form's workspace is the library's static array."""
    s = _stream(stream)
    check(lib.qmm_gdn_recurrence_noalloc(byref(y.h), byref(state_out.h), q.h, k.h, v.h, g.h, beta.h, state.h,
                                         y_dtype, s.h), "gdn_recurrence_noalloc")
    return y, state_out


def mlp_gate_up_silu(x: Array, w_gate: Array, s_gate: Array, w_up: Array, s_up: Array, mode: str, *,
                     group_size=None, bits=None, out: Array | None = None, stream: Stream | None = None) -> Array:
    """silu(x @ deq(Wg).T) * (x @ deq(Wu).T) (src/model.zig:905-913), fused for decode shapes."""
    res = out if out is not None else Array()
    s = _stream(stream)
    check(lib.qmm_mlp_gate_up_silu(byref(res.h), x.h, w_gate.h, s_gate.h, w_up.h, s_up.h, opt_int(group_size),
                                   opt_int(bits), mode.encode(), s.h), "mlp_gate_up_silu")
    return res


def quantized_matmul_group(x: Array, ws, scales, mode: str, *, group_size=None, bits=None, outs=None,
                           stream: Stream | None = None) -> list:
    """[x @ deq(w_i).T for each (w_i, scales_i)]: projections of one x (src/model.zig:1066-1074,
    :929-944), one launch when the matrices lie back to back in memory."""
    n = len(ws)
    assert len(scales) == n
    res = list(outs) if outs is not None else [Array() for _ in range(n)]
    hs = (qmm_array * n)(*[r.h for r in res])
    wv = (qmm_array * n)(*[w.h for w in ws])
    sv = (qmm_array * n)(*[sc.h for sc in scales])
    s = _stream(stream)
    rc = lib.qmm_quantized_matmul_group(hs, n, x.h, wv, sv, opt_int(group_size), opt_int(bits), mode.encode(), s.h)
    for r, h in zip(res, hs):
        r.h = h
    check(rc, "quantized_matmul_group")
    return res


def infer_quant_spec_json(header: str):
    b = header.encode()
    spec = qmm_quant_spec()
    n = c_size_t(0)
    rc = lib.qmm_infer_quant_spec_json(b, len(b), byref(spec), byref(n))
    if rc:
        return WE.get(rc, rc)
    return {QUANT_NONE: "none", QUANT_MXFP8: "mxfp8", QUANT_NVFP4: "nvfp4"}[spec.mode], spec.group_size, spec.bits


def parse_header_json(header: str):
    b = header.encode()
    n = c_size_t(0)
    rc = lib.qmm_parse_header_json(b, len(b), byref(n))
    return WE.get(rc, rc) if rc else n.value


def sanitize_name(name: str):
    buf = ctypes.create_string_buffer(4096)
    rc = lib.qmm_sanitize_name(name.encode(), buf, 4096)
    return buf.value.decode() if rc == 1 else None


class WeightMap:
    def __init__(self, model_dir: str, stream: Stream | None = None):
        self.h = qmm_weight_map(None)
        s = _stream(stream)
        rc = lib.qmm_weights_load(byref(self.h), str(model_dir).encode(), s.h)
        if rc:
            raise QmmError(f"weights_load: {WE.get(rc, rc)}: {take_error()}")

    def get(self, name: str) -> Array | None:
        h = lib.qmm_weights_get(self.h, name.encode())
        if not h.ctx:
            return None
        a = Array(qmm_array(None))
        a.h = h
        a.free = lambda: None  # borrowed: the map owns it
        return a

    def __len__(self):
        return lib.qmm_weights_count(self.h)

    @property
    def quant(self):
        q = lib.qmm_weights_quant(self.h)
        return {QUANT_NONE: "none", QUANT_MXFP8: "mxfp8", QUANT_NVFP4: "nvfp4"}[q.mode], q.group_size, q.bits

    def named_linear_q(self, x: Array, name: str, stream: Stream | None = None) -> Array:
        res = Array()
        s = _stream(stream)
        rc = lib.qmm_named_linear_q(byref(res.h), self.h, x.h, name.encode(), s.h)
        if rc:
            raise QmmError(f"named_linear_q: {WE.get(rc, rc)}: {take_error()}")
        return res

    def named_linear_q_group(self, x: Array, names, stream: Stream | None = None) -> list:
        """Projections of one x by name, one grouped call when all are packed with scales."""
        n = len(names)
        res = [Array() for _ in range(n)]
        hs = (qmm_array * n)(*[r.h for r in res])
        nm = (c_char_p * n)(*[x_.encode() for x_ in names])
        s = _stream(stream)
        rc = lib.qmm_named_linear_q_group(hs, n, self.h, x.h, nm, s.h)
        for r, h in zip(res, hs):
            r.h = h
        if rc:
            raise QmmError(f"named_linear_q_group: {WE.get(rc, rc)}: {take_error()}")
        return res

    def mlp_forward_q(self, x: Array, gate: str, down: str, up: str, stream: Stream | None = None) -> Array:
        """mlpForwardQ (src/model.zig:905-915): down(silu(gate(x)) * up(x))."""
        res = Array()
        s = _stream(stream)
        rc = lib.qmm_mlp_forward_q(byref(res.h), self.h, x.h, gate.encode(), down.encode(), up.encode(), s.h)
        if rc:
            raise QmmError(f"mlp_forward_q: {WE.get(rc, rc)}: {take_error()}")
        return res

    def __del__(self):
        try:
            if self.h.ctx:
                lib.qmm_weights_free(self.h)
        except Exception:
            pass


def declared_symbols() -> list[str]:
    """Every function the public header declares."""
    import re

    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmm_[a-z0-9_]+)\s*\(", text)) - {"qmm_error_handler_func"})
