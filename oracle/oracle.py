"""ctypes wrapper over the C oracle (``oracle/qmm_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the CPU-baseline leg of ``bench.py``, and only as the checker.  The HIP
product path never imports this module.

The oracle restates ``mlx_quantized_matmul`` / ``mlx_dequantize`` /
``mlx_quantize`` as the reference binds them (src/mlx.zig:265, :274, :278) for
the two microscaling modes the reference serves (src/weights.zig:37-55):

* mxfp8: group 32, E4M3 elements packed 4 per uint32 (LSB first), E8M0 scales.
* nvfp4: group 16, E2M1 elements packed 8 per uint32 (LSB first), E4M3 scales.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

MODES = {"mxfp8": 0, "nvfp4": 1}
GROUP = {"mxfp8": 32, "nvfp4": 16}
BITS = {"mxfp8": 8, "nvfp4": 4}

_lib = None


def build() -> Path:
    """Compile liboracle.so with oracle/Makefile (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        u8, u16, f32, f64, i32, i64, vp = (ctypes.c_uint8, ctypes.c_uint16, ctypes.c_float,
                                            ctypes.c_double, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_void_p)
        for name, res, args in [
            ("oracle_e4m3_to_f32", f32, [u8]),
            ("oracle_e8m0_to_f32", f32, [u8]),
            ("oracle_e2m1_to_f32", f32, [u8]),
            ("oracle_bf16_to_f32", f32, [u16]),
            ("oracle_f64_to_bf16", u16, [f64]),
            ("oracle_f32_to_bf16", u16, [f32]),
            ("oracle_e4m3_encode", u8, [f64]),
            ("oracle_e2m1_encode", u8, [f64]),
            ("oracle_dequant", None, [i32, vp, vp, i64, i64, vp]),
            ("oracle_dequant_bf16", None, [i32, vp, vp, i64, i64, vp]),
            ("oracle_dequant_f64", None, [i32, vp, vp, i64, i64, vp]),
            ("oracle_quantize", None, [i32, vp, i64, i64, vp, vp]),
            ("oracle_qmm", i32, [i32, i32, vp, i64, i64, vp, vp, i64, vp, i64, i32, vp, i32, i32]),
        ]:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- scalars
def e4m3_table() -> np.ndarray:
    return np.array([lib().oracle_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)


def e8m0_table() -> np.ndarray:
    return np.array([lib().oracle_e8m0_to_f32(i) for i in range(256)], dtype=np.float32)


def e2m1_table() -> np.ndarray:
    return np.array([lib().oracle_e2m1_to_f32(i) for i in range(16)], dtype=np.float32)


def f64_to_bf16_bits(v: float) -> int:
    return int(lib().oracle_f64_to_bf16(float(v)))


def f64_to_bf16_bits_vec(v: np.ndarray) -> np.ndarray:
    """Round float64 -> bf16 bits once, nearest-even (vectorised oracle_f64_to_bf16):
    8 significant bits via frexp / rint (exact in float64), subnormals on the
    2^-133 grid, overflow to inf, NaN -> 0x7FC0."""
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)
    q = np.ldexp(np.rint(np.ldexp(m, 8)), e - 8)
    q = np.where(np.abs(v) < 2.0 ** -126, np.ldexp(np.rint(np.ldexp(v, 133)), -133), q)
    with np.errstate(over="ignore", invalid="ignore"):
        f = q.astype(np.float32)
    return np.where(np.isnan(v), np.uint16(0x7FC0), f32_to_bf16_bits(f))


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 -> bf16 bits, nearest-even (vectorised; NaN -> 0x7FC0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


# ---------------------------------------------------------------- dequant / quantize
def dequant(mode: str, w: np.ndarray, s: np.ndarray, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    N = w.shape[0]
    out = np.empty((N, K), dtype=np.float32)
    lib().oracle_dequant(MODES[mode], _ptr(w), _ptr(s), N, K, _ptr(out))
    return out


def dequant_f64(mode: str, w: np.ndarray, s: np.ndarray, K: int) -> np.ndarray:
    """The exact dequantized weights (elem * scale in float64; never overflows)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    N = w.shape[0]
    out = np.empty((N, K), dtype=np.float64)
    lib().oracle_dequant_f64(MODES[mode], _ptr(w), _ptr(s), N, K, _ptr(out))
    return out


def dequant_bf16(mode: str, w: np.ndarray, s: np.ndarray, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    N = w.shape[0]
    out = np.empty((N, K), dtype=np.uint16)
    lib().oracle_dequant_bf16(MODES[mode], _ptr(w), _ptr(s), N, K, _ptr(out))
    return out


def quantize(mode: str, w: np.ndarray):
    """w: float32 [N, K] (bf16-valued inputs are exact in f32) -> (packed u32, scales u8)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    assert K % GROUP[mode] == 0
    wq = np.empty((N, K * BITS[mode] // 32), dtype=np.uint32)
    s = np.empty((N, K // GROUP[mode]), dtype=np.uint8)
    lib().oracle_quantize(MODES[mode], _ptr(w), N, K, _ptr(wq), _ptr(s))
    return wq, s


# ---------------------------------------------------------------- qmm
def qmm(mode: str, x: np.ndarray, w: np.ndarray, s: np.ndarray, *, x_is_bf16: bool = True,
        cols: np.ndarray | None = None, out: str = "bf16", f32acc: bool = False,
        threads: int | None = None) -> np.ndarray:
    """y = x @ deq(W).T.

    x: [M, K] as bf16 bits (uint16, ``x_is_bf16``) or float32.
    cols: optional output-column subset (int64 indices into N).
    out: "bf16" (uint16 bits, RNE of the double sum) or "f32".
    f32acc: f32 weights and fp32 accumulation (the CPU-baseline form) instead of
    exact weights and a double sum (the parity form: a weight is elem * scale
    exactly, NaN codes and scales make it NaN, and only the final sum rounds).
    """
    x = np.ascontiguousarray(x, dtype=np.uint16 if x_is_bf16 else np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] * 32 // BITS[mode] == K, (w.shape, K)
    assert s.shape == (N, K // GROUP[mode]), (s.shape, N, K)
    if cols is not None:
        cols = np.ascontiguousarray(cols, dtype=np.int64)
        ncols = cols.shape[0]
        cptr = _ptr(cols)
    else:
        ncols, cptr = N, None
    y = np.empty((M, ncols), dtype=np.uint16 if out == "bf16" else np.float32)
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    lib().oracle_qmm(MODES[mode], 0 if x_is_bf16 else 1, _ptr(x), M, K, _ptr(w), _ptr(s), N, cptr,
                     ncols, 0 if out == "bf16" else 1, _ptr(y), 1 if f32acc else 0, threads)
    return y


# ---------------------------------------------------------------- tolerance
def check_tolerance(y: np.ndarray, y_ref: np.ndarray, *, rel_fro: float = 1e-3, ulps: float = 4.0):
    """Compare bf16 outputs (as float32 values) against the oracle's bf16 outputs.

    rel Frobenius error <= rel_fro, and per row m: max_n |y - y_ref| <= ulps *
    ulp(max_n |y_ref[m, n]|), ulp(v) = 2^(floor(log2 v) - 7).
    Returns (ok, rel_fro_err, worst_ulp_ratio).
    """
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    if not np.array_equal(np.isnan(y), np.isnan(r)):
        return False, float("inf"), float("inf")
    y = np.nan_to_num(y)
    r = np.nan_to_num(r)
    den = np.linalg.norm(r)
    fro = float(np.linalg.norm(y - r) / den) if den > 0 else float(np.linalg.norm(y - r))
    worst = 0.0
    for m in range(r.shape[0]):
        scale = np.max(np.abs(r[m]))
        if scale == 0:
            err = np.max(np.abs(y[m])) if y.shape[1] else 0.0
            worst = max(worst, float("inf") if err > 0 else 0.0)
            continue
        ulp = 2.0 ** (np.floor(np.log2(scale)) - 7)
        worst = max(worst, float(np.max(np.abs(y[m] - r[m])) / ulp))
    return (fro <= rel_fro and worst <= ulps), fro, worst


def silu_mul_bf16(g_bits: np.ndarray, u_bits: np.ndarray) -> np.ndarray:
    """mlx-runner's MLP activation on bf16 arrays, op by op (src/model.zig:405-415
    silu = x * sigmoid(x), :451-456 mul; used by mlpForwardQ :905-915): each op's
    result is rounded to bf16 (nearest-even).  sigmoid is evaluated in float64.
    Inputs and output are bf16 bit patterns (uint16)."""
    g = bf16_bits_to_f32(g_bits).astype(np.float64)
    u = bf16_bits_to_f32(u_bits).astype(np.float64)
    r = lambda v: bf16_bits_to_f32(f64_to_bf16_bits_vec(v)).astype(np.float64)
    with np.errstate(over="ignore"):
        sg = r(1.0 / (1.0 + np.exp(-g)))
    sl = r(g * sg)
    return f64_to_bf16_bits_vec(sl * u)
