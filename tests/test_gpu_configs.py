"""Parity at the benchmark's full shapes.

For each configured workload the weights are generated and quantized on the
GPU.  Every output buffer is filled with bf16 NaN (0xFFFF) before the call,
so an output element the kernels never write cannot pass.  The checks are
  * every element of every output is finite after the call,
  * the GPU quantizer is bit-exact against the oracle on sampled rows,
  * decode shapes (M <= 8): EVERY output column of every row is within
    tolerance of the oracle,
  * prefill shapes: every column of one row from each 256-row tile (the GEMM
    tile height), plus 64 sampled columns over all rows, within tolerance,
  * linearity: qmm(2x) == 2 qmm(x) bit-for-bit (power-of-two scaling commutes
    with every rounding in the path), and
  * determinism: a second call returns identical bits.

The lm_head shapes include M = 2 and 3, the rows logitsOf / mtpDraftLogits
take on the speculative-verify path (src/engine.zig:552, :660;
src/model.zig:1299-1310), and the dense bf16 lm_head of mxfp8 checkpoints
(src/model.zig:215-216) at its full [248320, 5120].
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
    "nvfp4_gateup_3x34816x5120": ("nvfp4", 3, 34816, 5120, 1.0),
    "nvfp4_down_1x5120x17408": ("nvfp4", 1, 5120, 17408, 0.5),
    "nvfp4_down_2x5120x17408": ("nvfp4", 2, 5120, 17408, 0.5),
    "nvfp4_down_3x5120x17408": ("nvfp4", 3, 5120, 17408, 0.5),
    "mxfp8_down_1x5120x17408": ("mxfp8", 1, 5120, 17408, 0.5),
    "mxfp8_down_3x5120x17408": ("mxfp8", 3, 5120, 17408, 0.5),
    "mxfp8_prefill_4096x17408x5120": ("mxfp8", 4096, 17408, 5120, 1.0),
    "nvfp4_lmhead_1x248320x5120": ("nvfp4", 1, 248320, 5120, 1.0),
    "nvfp4_lmhead_2x248320x5120": ("nvfp4", 2, 248320, 5120, 1.0),
    "nvfp4_lmhead_3x248320x5120": ("nvfp4", 3, 248320, 5120, 1.0),
    "nvfp4_lmhead_2048x248320x5120": ("nvfp4", 2048, 248320, 5120, 1.0),
}
TILE = 256  # rows of one prefill GEMM tile


def nan_filled(shape, dev):
    """A bf16 tensor whose every element is NaN (bit pattern 0xFFFF)."""
    y = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    y.view(torch.int16).fill_(-1)
    return y


def tile_rows(M):
    """Rows checked in full for a prefill shape: one per 256-row tile (at a
    different offset in each tile), the first and the last row."""
    r =[min(M - 1, t * TILE + (t * 97 + 13) % TILE) for t in range((M + TILE - 1) // TILE)]
    return np.unique(np.array(r + [0, M - 1], dtype=np.int64))


def assert_written(y, what):
    bad = int((~torch.isfinite(y)).sum().item())
    assert bad == 0, f"{what}: {bad} of {y.numel()} output elements not written (still NaN) or not finite"


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
    y = nan_filled((M, N), dev)
    Q.quantized_matmul(xa, wq, sc, mode, out=Q.Array.from_torch(y), stream=stream)
    x2 = (x.float() * 2).to(torch.bfloat16)  # exact
    y2 = nan_filled((M, N), dev)
    Q.quantized_matmul(Q.Array.from_torch(x2), wq, sc, mode, out=Q.Array.from_torch(y2), stream=stream)
    y3 = nan_filled((M, N), dev)
    Q.quantized_matmul(xa, wq, sc, mode, out=Q.Array.from_torch(y3), stream=stream)
    torch.cuda.synchronize()
    for t, what in ((y, "y"), (y2, "y(2x)"), (y3, "y again")):
        assert_written(t, what)
    assert torch.equal(y.view(torch.int16), y3.view(torch.int16)), "not deterministic"
    assert torch.equal((y.float() * 2).to(torch.bfloat16).view(torch.int16), y2.view(torch.int16)), "not linear"

    wq_h, s_h = wq.numpy(stream), sc.numpy(stream)
    rng = np.random.default_rng(0)
    qrows = np.unique(np.concatenate([[0, N - 1], rng.choice(N, size=62, replace=False)])).astype(np.int64)
    Wr = W[torch.from_numpy(qrows).to(dev)].float().cpu().numpy()
    rq, rs = O.quantize(mode, Wr)
    assert np.array_equal(wq_h[qrows], rq) and np.array_equal(s_h[qrows], rs), "quantizer differs from the oracle"
    del W
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)

    if M <= 8:
        # every column of every row
        ref = O.qmm(mode, xb, wq_h, s_h)
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref))
        print(f"[config] {name}: all {M}x{N} outputs: rel_fro={fro:.3e} max_ulp={worst:.2f}", flush=True)
        assert ok, (fro, worst)
        return

    # every column of one row per 256-row tile
    rows = tile_rows(M)
    ref = O.qmm(mode, np.ascontiguousarray(xb[rows]), wq_h, s_h)
    got = y[torch.from_numpy(rows).to(dev)].view(torch.int16).cpu().numpy().view(np.uint16)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref))
    print(f"[config] {name}: rows {len(rows)} x all {N} columns: rel_fro={fro:.3e} max_ulp={worst:.2f}", flush=True)
    assert ok, ("tile rows", fro, worst)
    # and sampled columns over every row
    cols = np.unique(np.concatenate([[0, N - 1], rng.choice(N, size=62, replace=False)])).astype(np.int64)
    ref = O.qmm(mode, xb, wq_h, s_h, cols=cols)
    got = y[:, torch.from_numpy(cols).to(dev)].view(torch.int16).cpu().numpy().view(np.uint16)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref))
    print(f"[config] {name}: all {M} rows x {len(cols)} columns: rel_fro={fro:.3e} max_ulp={worst:.2f}", flush=True)
    assert ok, ("column sample", fro, worst)


@pytest.mark.parametrize("M", [1, 3])
def test_full_size_dense_lmhead(M):
    """The dense bf16 lm_head of mxfp8 checkpoints (linear, src/model.zig:200-211,
    :215-216) at [248320, 5120]: every output against a float64 product on the host,
    rounded once to bf16."""
    N, K = 248320, 5120
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(4100 + M)
    W = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    y = nan_filled((M, N), dev)
    stream = Q.Stream.torch_current()
    Q.linear(Q.Array.from_torch(x), Q.Array.from_torch(W), out=Q.Array.from_torch(y), stream=stream)
    torch.cuda.synchronize()
    assert_written(y, "dense lm_head y")
    xf = x.float().cpu().numpy().astype(np.float64)
    ref = np.empty((M, N), np.float64)
    step = 16384
    for r0 in range(0, N, step):
        wc = W[r0:r0 + step].float().cpu().numpy().astype(np.float64)
        ref[:, r0:r0 + step] = xf @ wc.T
    refb = O.f64_to_bf16_bits_vec(ref)
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(refb))
    print(f"[config] dense lm_head M={M}: all {M}x{N} outputs: rel_fro={fro:.3e} max_ulp={worst:.2f}", flush=True)
    assert ok, (fro, worst)
