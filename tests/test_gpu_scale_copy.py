"""The prefill GEMMs' tile-major scale copy: ordering across streams and its lifetime.

The first prefill call (M > 8) with a scales handle makes a tile-major copy of the
scales and keeps it with the handle.  Calls on other streams, issued with no
synchronisation after that first call, must read the finished copy; freeing the
handle (or the weight map that owns it) frees the copy.  The reference runs one
inference stream and reads results after eval (src/mlx.zig:265, AGENTS.md:69-70);
the several-stream cases are this library's own contract for its callers.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import qmm as Q
from test_gpu_loader import make_checkpoint

pytestmark = pytest.mark.gpu

GROUP = {"mxfp8": 32, "nvfp4": 16}


def round256(v):
    return (v + 255) // 256 * 256


def fresh_view(a):
    """A new handle on the same device bytes (so it holds no scale copy yet)."""
    shape = (ctypes.c_int * len(a.shape))(*a.shape)
    h = Q.lib.qmm_array_new_device(ctypes.c_void_p(a.ptr), shape, len(a.shape), a.dtype)
    assert h.ctx
    return Q.Array(h, keepalive=a)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_first_prefill_on_two_streams_with_a_fresh_scales_handle(mode):
    """Stream A is kept busy by a long (bounded) matmul chain; the first prefill call with a
    fresh scales handle is issued on A, and the same call on stream B right after it with no
    synchronisation.  B's output (NaN-filled beforehand) equals the serial result bit for bit,
    and the copy's bytes are accounted to the handle and returned when it is freed."""
    import torch

    M, N, K = 300, 1536, 2048
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(303)
    W = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    wq, sc = Q.quantize(Q.Array.from_torch(W), mode)
    serial = Q.quantized_matmul(Q.Array.from_torch(x), wq, sc, mode).numpy().view(np.int16)
    torch.cuda.synchronize()

    before = Q.lib.qmm_scale_copy_bytes()
    fresh = fresh_view(sc)
    big = torch.randn((4096, 4096), generator=g, device=dev)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    ya = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    yb = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        acc = big
        for _ in range(8):  # a few ms of work queued ahead of the first prefill call
            acc = torch.tanh(acc @ big)
        Q.quantized_matmul(Q.Array.from_torch(x), wq, fresh, mode, out=Q.Array.from_torch(ya),
                           stream=Q.Stream.torch_current())
    with torch.cuda.stream(sb):
        Q.quantized_matmul(Q.Array.from_torch(x), wq, fresh, mode, out=Q.Array.from_torch(yb),
                           stream=Q.Stream.torch_current())
    torch.cuda.synchronize()
    assert np.array_equal(ya.view(torch.int16).cpu().numpy(), serial)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy(), serial)
    assert Q.lib.qmm_scale_copy_bytes() == before + round256(N) * K // GROUP[mode]
    fresh.free()
    assert Q.lib.qmm_scale_copy_bytes() == before
    assert Q.take_error() is None
    # and the serial bits are the right ones
    cols = np.arange(0, N, 5)
    ref = O.qmm(mode, x.view(torch.int16).cpu().numpy().view(np.uint16), wq.numpy(), sc.numpy(), cols=cols)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(serial.view(np.uint16)[:, cols]), O.bf16_bits_to_f32(ref),
                                       rel_fro=1e-3, ulps=4.0)
    assert ok, (fro, worst)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_first_prefill_from_four_threads_at_once(mode):
    """Four host threads, each on its own stream, make the first prefill call with one fresh
    scales handle at the same moment: one copy is made, and every output equals the serial
    result bit for bit."""
    import threading

    import torch

    M, N, K = 260, 1024, 1024
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(304)
    W = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    wq, sc = Q.quantize(Q.Array.from_torch(W), mode)
    serial = Q.quantized_matmul(Q.Array.from_torch(x), wq, sc, mode).numpy().view(np.int16)
    torch.cuda.synchronize()
    before = Q.lib.qmm_scale_copy_bytes()
    fresh = fresh_view(sc)
    barrier = threading.Barrier(4)
    outs, errors = {}, []

    def worker(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
                barrier.wait()
                Q.quantized_matmul(Q.Array.from_torch(x), wq, fresh, mode, out=Q.Array.from_torch(y),
                                   stream=Q.Stream.torch_current())
                outs[t] = y
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t, y in outs.items():
        assert np.array_equal(y.view(torch.int16).cpu().numpy(), serial), t
    assert Q.lib.qmm_scale_copy_bytes() == before + round256(N) * K // GROUP[mode]
    fresh.free()
    assert Q.lib.qmm_scale_copy_bytes() == before


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_weight_map_frees_its_scale_copies(tmp_path, mode):
    """Prefill calls through a loaded weight map attach scale copies to the map's scales
    handles; freeing the map frees them (load -> prefill -> free leaves nothing behind)."""
    import gc

    N, K = 48, 256
    before = Q.lib.qmm_scale_copy_bytes()
    pre, quant, _, _ = make_checkpoint(tmp_path, mode, N=N, K=K)
    for cycle in range(2):
        wmap = Q.WeightMap(str(tmp_path))
        xb = O.f32_to_bf16_bits(np.random.default_rng(9 + cycle).standard_normal((20, K)).astype(np.float32))
        x = Q.Array.from_numpy(xb, Q.BFLOAT16)
        for proj in ("mlp.down_proj", "mlp.up_proj"):
            y = wmap.named_linear_q(x, pre + proj + ".weight").numpy()
            ref = O.qmm(mode, xb, *quant[proj])
            ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(ref), rel_fro=1e-3, ulps=4.0)
            assert ok, (proj, fro, worst)
        assert Q.lib.qmm_scale_copy_bytes() == before + 2 * round256(N) * K // GROUP[mode]
        del wmap
        gc.collect()
        assert Q.lib.qmm_scale_copy_bytes() == before, cycle
