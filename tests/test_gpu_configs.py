"""Parity at the benchmark's full shapes.

For each configured workload the weights are generated and quantized on the
GPU; the checks are
  * the GPU quantizer is bit-exact against the oracle on sampled rows,
  * y on sampled output columns is within tolerance of the oracle (all M rows),
  * linearity: qmm(2x) == 2 qmm(x) bit-for-bit (power-of-two scaling commutes
    with every rounding in the path), and
  * determinism: a second call returns identical bits.
"""
import zlib

import numpy as np
import pytest
import torch

import oracle as O
import qmm as Q

pytestmark = pytest.mark.gpu

CONFIGS = {
    "mxfp8_gemv_1x5120x5120": ("mxfp8", 1, 5120, 5120, 1.0),
    "nvfp4_gateup_1x34816x5120": ("nvfp4", 1, 34816, 5120, 1.0),
    "nvfp4_down_1x5120x17408": ("nvfp4", 1, 5120, 17408, 0.5),
    "nvfp4_down_2x5120x17408": ("nvfp4", 2, 5120, 17408, 0.5),
    "nvfp4_down_3x5120x17408": ("nvfp4", 3, 5120, 17408, 0.5),
    "mxfp8_prefill_4096x17408x5120": ("mxfp8", 4096, 17408, 5120, 1.0),
    "nvfp4_lmhead_1x248320x5120": ("nvfp4", 1, 248320, 5120, 1.0),
    "nvfp4_lmhead_2048x248320x5120": ("nvfp4", 2048, 248320, 5120, 1.0),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_full_size_config(name):
    mode, M, N, K, xscale = CONFIGS[name]
    print(f"[config] {name}", flush=True)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(zlib.crc32(name.encode()))
    W = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = (torch.randn((M, K), generator=g, device=dev) * xscale).to(torch.bfloat16)
    stream = Q.Stream.torch_current()
    wq, sc = Q.quantize(Q.Array.from_torch(W), mode, stream=stream)
    xa = Q.Array.from_torch(x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    Q.quantized_matmul(xa, wq, sc, mode, out=Q.Array.from_torch(y), stream=stream)
    x2 = (x.float() * 2).to(torch.bfloat16)  # exact
    y2 = torch.empty_like(y)
    Q.quantized_matmul(Q.Array.from_torch(x2), wq, sc, mode, out=Q.Array.from_torch(y2), stream=stream)
    y3 = torch.empty_like(y)
    Q.quantized_matmul(xa, wq, sc, mode, out=Q.Array.from_torch(y3), stream=stream)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y3.view(torch.int16)), "not deterministic"
    assert torch.equal((y.float() * 2).to(torch.bfloat16).view(torch.int16), y2.view(torch.int16)), "not linear"

    rng = np.random.default_rng(0)
    cols = np.unique(np.concatenate([[0, N - 1], rng.choice(N, size=62, replace=False)])).astype(np.int64)
    wq_h, s_h = wq.numpy(stream), sc.numpy(stream)
    Wr = W[torch.from_numpy(cols).to(dev)].float().cpu().numpy()
    rq, rs = O.quantize(mode, Wr)
    assert np.array_equal(wq_h[cols], rq) and np.array_equal(s_h[cols], rs), "quantizer differs from the oracle"
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.qmm(mode, xb, wq_h, s_h, cols=cols)
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)[:, cols]
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref))
    print(f"[config] {name}: rel_fro={fro:.3e} max_ulp={worst:.2f}", flush=True)
    assert ok, (fro, worst)
