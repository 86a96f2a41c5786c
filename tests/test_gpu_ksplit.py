"""Prefill GEMMs with fewer tiles than half the CUs: every tile's K steps split over
several blocks, whose fp32 partial sums a second kernel adds in K order.

These are the short prefill chunks (the last partial chunk, the tokens left after a
prefix-cache hit, src/engine.zig:364-382) and the narrow projections at full chunk
size (k_proj / v_proj, N = 1024, src/model.zig:940-944).  Bar as everywhere: the
oracle within rel Frobenius 1e-3 and 4 bf16 ulps of each row's scale; and two calls
give the same bits (the partials are summed in a fixed order).
"""
import numpy as np
import pytest

import oracle as O
import qmm as Q

pytestmark = pytest.mark.gpu

TOL = dict(rel_fro=1e-3, ulps=4.0)


def _case(mode, M, N, K, seed):
    import torch

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    W = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    wq, sc = Q.quantize(Q.Array.from_torch(W), mode)
    return x, wq, sc


# (mode, M, N, K): 128-row tiles (nvfp4, M <= 128) and 256-row tiles, one to 68 tile columns;
# then x of at most 128 rows with more tiles than block slots (whole tiles of the short
# height, stored without partial sums) or between half and all of them (nvfp4 M = 9 at the
# fused gate+up width: 136 tiles of 64 rows, split 3 ways)
SHAPES = [
    ("nvfp4", 16, 17408, 5120), ("nvfp4", 100, 5120, 5120), ("nvfp4", 128, 12288, 5120),
    ("nvfp4", 129, 4096, 5120), ("nvfp4", 256, 17408, 5120), ("nvfp4", 40, 1000, 1024),
    ("mxfp8", 16, 17408, 5120), ("mxfp8", 64, 5120, 6144), ("mxfp8", 256, 17408, 5120),
    ("mxfp8", 300, 1000, 1024), ("mxfp8", 9, 2048, 10240),
    ("nvfp4", 9, 34816, 5120), ("nvfp4", 16, 70001, 1024), ("nvfp4", 100, 40000, 1024),
    ("mxfp8", 20, 40000, 1024), ("mxfp8", 128, 34816, 1024),
]


@pytest.mark.parametrize("mode,M,N,K", SHAPES)
def test_split_tiles_match_oracle_and_repeat_bit_for_bit(mode, M, N, K):
    import torch

    x, wq, sc = _case(mode, M, N, K, 500 + M + N % 101)
    ys = []
    for _ in range(2):
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        Q.quantized_matmul(Q.Array.from_torch(x), wq, sc, mode, out=Q.Array.from_torch(y))
        ys.append(y)
    torch.cuda.synchronize()
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))
    assert torch.isfinite(ys[0].float()).all()
    cols = np.arange(0, N, 1 if N * M <= 1 << 20 else 7)
    ref = O.qmm(mode, x.view(torch.int16).cpu().numpy().view(np.uint16), wq.numpy(), sc.numpy(), cols=cols)
    got = ys[0].view(torch.int16).cpu().numpy().view(np.uint16)[:, cols]
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref), **TOL)
    assert ok, (fro, worst)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_narrow_projection_at_full_chunk(mode):
    """k_proj at a 4096-token chunk: 64 tiles of 256 x 256, so each tile's K runs on 4 blocks."""
    import torch

    M, N, K = 4096, 1024, 5120
    x, wq, sc = _case(mode, M, N, K, 777)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    Q.quantized_matmul(Q.Array.from_torch(x), wq, sc, mode, out=Q.Array.from_torch(y))
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    rows = np.r_[0:4096:61, 4095]
    xr = x[torch.from_numpy(rows).cuda()].contiguous()
    ref = O.qmm(mode, xr.view(torch.int16).cpu().numpy().view(np.uint16), wq.numpy(), sc.numpy())
    got = y[torch.from_numpy(rows).cuda()].view(torch.int16).cpu().numpy().view(np.uint16)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(ref), **TOL)
    assert ok, (fro, worst)
