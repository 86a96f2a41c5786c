"""Error classes surfaced at the checkpoints (src/mlx.zig:737-868) from real failures
on the GPU, through the C ABI.

A device allocation far larger than the GPU's memory fails inside an op; the op
returns non-zero without launching anything, the latched message is classified as
a memory error, and qmm_check_error() reports QMM_ERR_OOM once (the reference's
OutOfMemory class), then 0.
"""
from ctypes import byref, c_int, c_void_p

import pytest
import torch

import qmm as Q

pytestmark = pytest.mark.gpu


def test_failed_allocation_reports_out_of_memory():
    free, total = torch.cuda.mem_get_info()
    buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")  # what the handles point at
    N, K = 1 << 20, 1 << 22  # the dequantized f32 result would take N * K * 4 = 16 TiB
    assert N * K * 4 > 16 * total
    # packed nvfp4 words [N, K / 8] and scales [N, K / 16] over the small buffer: the op
    # checks shapes, fails to allocate its result and returns before any kernel runs
    w = Q.lib.qmm_array_new_device(c_void_p(buf.data_ptr()), (c_int * 2)(N, K // 8), 2, Q.UINT32)
    s = Q.lib.qmm_array_new_device(c_void_p(buf.data_ptr()), (c_int * 2)(N, K // 16), 2, Q.UINT8)
    Q.lib.qmm_reset_faults_for_test()
    res = Q.qmm_array(None)
    st = Q.Stream.torch_current()
    rc = Q.lib.qmm_dequantize(byref(res), w, s, Q.qmm_array(None), Q.opt_int(), Q.opt_int(), b"nvfp4",
                              Q.qmm_array(None), Q.qmm_optional_dtype(Q.FLOAT32, True), st.h)
    try:
        assert rc != 0 and not res.ctx
        assert Q.lib.qmm_peek_error_name() == b"OutOfMemory"
        assert Q.lib.qmm_check_error() == Q.ERR_OOM
        assert Q.lib.qmm_check_error() == 0
        torch.cuda.synchronize()  # nothing was launched; the device is unaffected
        assert int(buf.sum().item()) == 0
    finally:
        Q.lib.qmm_array_free(w)
        Q.lib.qmm_array_free(s)


@pytest.mark.parametrize("mode,M", [("nvfp4", 1), ("mxfp8", 3), ("nvfp4", 40), ("mxfp8", 300)])
def test_error_left_by_other_code_is_not_an_op_failure(mode, M):
    """A HIP error the caller's own code left in the runtime (here hipSetDevice on a device
    that does not exist, its return code ignored) is not an error of the next op: the op
    succeeds, its result is right and nothing is latched."""
    import ctypes

    import numpy as np

    import oracle as O

    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch and the library share
    K, N = 1024, 512
    rng = np.random.default_rng(61 + M)
    wq, s = O.quantize(mode, O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.standard_normal((N, K)) * 0.02)))
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x, w, sc = Q.Array.from_numpy(xb, Q.BFLOAT16), Q.Array.from_numpy(wq, Q.UINT32), Q.Array.from_numpy(s, Q.UINT8)
    torch.cuda.synchronize()
    Q.lib.qmm_reset_faults_for_test()
    assert hip.hipSetDevice(ctypes.c_int(4096)) != 0  # leaves hipErrorInvalidDevice for this thread
    y = Q.quantized_matmul(x, w, sc, mode).numpy()
    assert Q.take_error() is None
    assert Q.lib.qmm_check_error() == 0
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(O.qmm(mode, xb, wq, s)),
                                       rel_fro=1e-3, ulps=4.0)
    assert ok, (fro, worst)
