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
