"""Host-side tests of the C ABI (no GPU work): exports, argument validation,
the error latch and the fault counters.

Mirrors the reference's error-path tests (src/mlx.zig:881-972) and the
argument rules of mlx_quantized_matmul as the reference uses it
(src/model.zig:244-260, src/weights.zig:37-55).
"""
import ctypes
import os
import subprocess
from ctypes import byref, c_int, c_void_p

import pytest

import qmm as Q

FAKE = 0x10000  # a never-dereferenced device address: validation fails before any launch


def _arr(shape, dtype, ptr=FAKE):
    sh = (c_int * max(len(shape), 1))(*shape)
    a = Q.lib.qmm_array_new_device(c_void_p(ptr), sh, len(shape), dtype)
    assert a.ctx
    return a


@pytest.fixture(autouse=True)
def _clean_latch():
    Q.lib.qmm_reset_faults_for_test()
    Q.lib.qmm_fault_arm(0)
    yield
    Q.lib.qmm_reset_faults_for_test()
    Q.lib.qmm_fault_arm(0)


def test_library_exports_every_declared_symbol():
    declared = Q.declared_symbols()
    assert len(declared) >= 40
    out = subprocess.run(["nm", "-D", "--defined-only", str(Q.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        assert getattr(Q.lib, s) is not None


def test_library_carries_gfx950_code_objects():
    blob = Q.LIB_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"amdgcn-amd-amdhsa--gfx942" not in blob


def _qmm_call(res, x, w, s, *, biases=None, transpose=True, gs=None, bits=None, mode=b"nvfp4"):
    return Q.lib.qmm_quantized_matmul(byref(res), x, w, s, biases or Q.qmm_array(None), transpose,
                                      Q.opt_int(gs), Q.opt_int(bits), mode, Q.qmm_stream(None))


@pytest.mark.parametrize("case,needle", [
    ("mode", "Unsupported quantization mode 'affine'"),
    ("bits", "requires bits 4"),
    ("group", "requires group_size 16"),
    ("biases", "takes no biases"),
    ("transpose", "transpose_w = true"),
    ("k_mismatch", "does not match the weight's K"),
    ("scales_shape", "scales shape"),
    ("w_dtype", "2D uint32"),
    ("x_dtype", "bfloat16 or float32"),
])
def test_quantized_matmul_rejects_bad_arguments(case, needle):
    N, K = 8, 64
    x = _arr([2, K], Q.BFLOAT16)
    w = _arr([N, K // 8], Q.UINT32)
    s = _arr([N, K // 16], Q.UINT8)
    kw = {}
    if case == "mode":
        kw["mode"] = b"affine"
    elif case == "bits":
        kw["bits"] = 8
    elif case == "group":
        kw["gs"] = 32
    elif case == "biases":
        kw["biases"] = _arr([N, K // 16], Q.BFLOAT16)
    elif case == "transpose":
        kw["transpose"] = False
    elif case == "k_mismatch":
        x = _arr([2, K + 16], Q.BFLOAT16)
    elif case == "scales_shape":
        s = _arr([N, K // 32], Q.UINT8)
    elif case == "w_dtype":
        w = _arr([N, K // 8], Q.UINT8)
    elif case == "x_dtype":
        x = _arr([2, K], Q.FLOAT16)
    res = Q.qmm_array(None)
    rc = _qmm_call(res, x, w, s, **kw)
    assert rc != 0
    assert Q.lib.qmm_error_pending()
    assert Q.lib.qmm_peek_error_name() == b"MlxFailure"
    msg = Q.take_error()
    assert needle in msg, msg
    assert not res.ctx  # nothing allocated on failure


def test_defaults_and_shape_inference_without_launch():
    """group/bits default by mode; an empty M needs no device work (src/weights.zig:37-55)."""
    for mode, g, bits in ((b"mxfp8", 32, 8), (b"nvfp4", 16, 4)):
        N, K = 48, 5120
        x = _arr([1, 0, K], Q.BFLOAT16)
        w = _arr([N, K * bits // 32], Q.UINT32)
        s = _arr([N, K // g], Q.UINT8)
        y = _arr([1, 0, N], Q.BFLOAT16, ptr=FAKE * 2)  # exact output shape -> written in place
        res = Q.qmm_array(y.ctx)
        assert _qmm_call(res, x, w, s, mode=mode) == 0
        assert _qmm_call(res, x, w, s, gs=g, bits=bits, mode=mode) == 0
        assert res.ctx == y.ctx
        assert not Q.lib.qmm_error_pending()


def test_fault_counter_fails_the_kth_succeeding_op():
    """src/mlx.zig:562-595: arm(k) makes the k-th succeeding checked op report failure."""
    N, K = 16, 64
    x = _arr([0, K], Q.BFLOAT16)
    w = _arr([N, K // 8], Q.UINT32)
    s = _arr([N, K // 16], Q.UINT8)
    res = Q.qmm_array(_arr([0, N], Q.BFLOAT16).ctx)
    before = Q.lib.qmm_op_count()
    Q.lib.qmm_fault_arm(3)
    assert _qmm_call(res, x, w, s) == 0
    assert _qmm_call(res, x, w, s, mode=b"bad") != 0  # failing ops are not counted
    Q.take_error()
    assert _qmm_call(res, x, w, s) == 0
    assert not Q.lib.qmm_fault_did_fire()
    assert _qmm_call(res, x, w, s) != 0  # third success -> injected failure
    assert Q.lib.qmm_fault_did_fire()
    assert res.ctx  # the out handle stays valid and freeable
    assert _qmm_call(res, x, w, s) == 0  # disarmed after firing
    assert Q.lib.qmm_op_count() - before == 5


def test_memory_errors_are_classified():
    """src/mlx.zig:881-889, plus HIP's out-of-memory name."""
    isMem = lambda m: Q.lib.qmm_error_is_memory(m.encode())  # noqa: E731
    assert isMem("[METAL] Command buffer execution failed: Insufficient Memory (kIOGPUCommandBufferCallbackErrorOutOfMemory). at transforms.cpp:15")
    assert isMem("[malloc] Unable to allocate 8589934592 bytes.")
    assert isMem("[metal::malloc] Resource limit (128000) exceeded.")
    assert isMem("[metal::malloc] Attempting to allocate 99 bytes which is greater than the maximum allowed buffer size of 5 bytes.")
    assert isMem("[quantized_matmul] hipErrorOutOfMemory: out of memory")
    assert not isMem("[slice_update] Invalid slice sizes.")
    assert not isMem("[matmul] Last dimension of first input must match.")


def test_latch_first_error_wins_and_is_consumed_once():
    """src/mlx.zig:891-906."""
    assert not Q.lib.qmm_error_pending()
    assert Q.lib.qmm_check_error() == 0
    Q.lib.qmm_latch_error_for_test(b"[METAL] Command buffer execution failed: Insufficient Memory. at transforms.cpp:15")
    assert Q.lib.qmm_error_pending()
    Q.lib.qmm_latch_error_for_test(b"[slice_update] Invalid slice sizes.")
    assert Q.lib.qmm_check_error() == Q.ERR_OOM
    assert not Q.lib.qmm_error_pending()
    assert Q.lib.qmm_check_error() == 0
    Q.lib.qmm_latch_error_for_test(b"[matmul] Last dimension of first input must match.")
    assert Q.lib.qmm_check_error() == Q.ERR_FAILURE
    assert not Q.lib.qmm_error_pending()


def test_peek_names_the_class_without_consuming():
    """src/mlx.zig:936-953."""
    assert Q.lib.qmm_peek_error_name() is None
    Q.lib.qmm_latch_error_for_test(b"[METAL] Command buffer execution failed: Insufficient Memory. at transforms.cpp:15")
    assert Q.lib.qmm_peek_error_name() == b"OutOfMemory"
    assert Q.lib.qmm_peek_error_name() == b"OutOfMemory"
    assert Q.lib.qmm_error_pending()
    assert Q.lib.qmm_check_error_decode() == Q.ERR_OOM
    assert Q.lib.qmm_peek_error_name() is None
    Q.lib.qmm_latch_error_for_test(b"[matmul] Last dimension of first input must match.")
    assert Q.lib.qmm_peek_error_name() == b"MlxFailure"
    assert Q.lib.qmm_check_error_decode() == Q.ERR_FAILURE


def test_decode_failure_is_attributed_to_the_decode_checkpoint():
    """src/mlx.zig:955-972."""
    assert Q.lib.qmm_check_error() == 0
    assert Q.lib.qmm_check_error_decode() == 0
    Q.lib.qmm_latch_error_for_test(b"[METAL] Command buffer execution failed: Insufficient Memory. at transforms.cpp:15")
    assert Q.lib.qmm_check_error_decode() == Q.ERR_OOM
    assert not Q.lib.qmm_error_pending()
    for _ in range(3):
        assert Q.lib.qmm_check_error() == 0
    assert Q.lib.qmm_check_error_decode() == 0


def test_env_fault_fires_once_at_the_nth_checkpoint(monkeypatch):
    """MLX_SERVE_MLX_FAULT_CHUNK / _STEP analogue (src/mlx.zig:807-868)."""
    monkeypatch.setenv("QMM_FAULT_CHUNK", "3")
    monkeypatch.setenv("QMM_FAULT_STEP", "2")
    Q.lib.qmm_reset_faults_for_test()
    assert Q.lib.qmm_check_error() == 0
    assert Q.lib.qmm_check_error() == 0
    assert Q.lib.qmm_check_error() == Q.ERR_OOM
    assert Q.lib.qmm_check_error() == 0  # disarmed
    assert Q.lib.qmm_check_error_decode() == 0
    assert Q.lib.qmm_check_error_decode() == Q.ERR_OOM
    assert Q.lib.qmm_check_error_decode() == 0


def test_error_handler_sees_every_message():
    seen = []
    cb = Q.ERROR_HANDLER(lambda msg, data: seen.append(msg.decode()))
    Q.lib.qmm_set_error_handler(cb, None, None)
    try:
        Q.lib.qmm_latch_error_for_test(b"first")
        Q.lib.qmm_latch_error_for_test(b"second")
        assert seen == ["first", "second"]
        buf = ctypes.create_string_buffer(64)
        assert Q.lib.qmm_take_error(buf, 64) == 5 and buf.value == b"first"
    finally:
        Q.lib.qmm_set_error_handler(Q.ERROR_HANDLER(0), None, None)
