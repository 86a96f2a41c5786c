"""Grouped projections of one x (qmm_quantized_matmul_group, qmm_named_linear_q_group).

The GDN layer's in_proj_qkv / z / b / a (src/model.zig:1066-1074) and attention's
q / k / v (:929-944) are consecutive qlinear calls on one x.  A grouped call runs
them as one matrix when they lie back to back in memory.  Checks:
  * every part against the oracle's qmm of the same bytes, at the qmm bar, for
    matrices back to back (one launch, counted), given in any order, and apart
    (one call per matrix);
  * part boundaries inside a row block and inside a workgroup's range (ragged
    parts of 3..1000 rows);
  * where the one launch and the single calls pick the same kernel family, the
    grouped parts equal the single calls bit for bit;
  * at prefill sizes one GEMM over the stacked matrices, whose epilogue and split-tile
    reduce store each column to its part;
  * the loader places a layer's group back to back across shards, and
    named_linear_q_group on it equals named_linear_q per name.
"""
import json

import numpy as np
import pytest

import oracle as O
import qmm as Q
from test_gpu_loader import write_safetensors

pytestmark = pytest.mark.gpu

TOL = dict(rel_fro=1e-3, ulps=4.0)


def bf16(a):
    return O.f32_to_bf16_bits(np.asarray(a, np.float32))


def bf16_round(a):
    """float32 -> nearest bf16 value (ties to even), as float32; finite inputs."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


_QUANT = {}


def quantized_rows(mode, rows, K, seed):
    key = (mode, tuple(rows), K, seed)
    if key not in _QUANT:
        rng = np.random.default_rng(seed)
        W = bf16_round(rng.standard_normal((sum(rows), K), dtype=np.float32) * np.float32(0.02))
        _QUANT[key] = O.quantize(mode, W)
    return _QUANT[key]


def device_group(mode, rows, K, seed):
    """Quantized matrices of `rows` rows each, carved back to back from one allocation.
    Returns (torch buffers, [(w_i, s_i) Arrays], [(wq_i, s_i) numpy])."""
    import torch

    wq, s = quantized_rows(mode, rows, K, seed)
    wt = torch.from_numpy(wq.view(np.int32)).cuda()
    st = torch.from_numpy(s).cuda()
    arrs, host, r0 = [], [], 0
    for n in rows:
        arrs.append((Q.Array.from_torch(wt[r0:r0 + n], dtype=Q.UINT32), Q.Array.from_torch(st[r0:r0 + n])))
        host.append((wq[r0:r0 + n], s[r0:r0 + n]))
        r0 += n
    return (wt, st), arrs, host


def check_parts(mode, xb, outs, host, what):
    for i, (y, (wq, s)) in enumerate(zip(outs, host)):
        ref = O.qmm(mode, xb, wq, s)
        yv = y.numpy()
        assert yv.shape == ref.shape, (what, i, yv.shape, ref.shape)
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(yv), O.bf16_bits_to_f32(ref), **TOL)
        assert ok, (what, i, fro, worst)


GROUPS = {
    "gdn_in_proj": (10240, 6144, 48, 48),     # qkv, z, b, a at the model's sizes
    "attn_qkv": (12288, 1024, 1024),          # q, k, v
    "ragged_small": (1000, 37, 530, 3),       # part boundaries inside row blocks (bf16 GEMV)
    "ragged_big": (12000, 4099, 301, 77),     # ... and on the MFMA kernels at M = 1
    "five_wave": (2560, 1280, 1280),          # 5120 rows: the bf16 GEMV's 5-wave workgroups at M = 1
}


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("group", sorted(GROUPS))
def test_group_back_to_back_one_launch(mode, M, group):
    rows, K = GROUPS[group], 5120
    print(f"group {group} {mode} M={M}", flush=True)
    keep, arrs, host = device_group(mode, rows, K, seed=sorted(GROUPS).index(group))
    rng = np.random.default_rng(M)
    xb = bf16(rng.standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    before = Q.lib.qmm_group_launch_count()
    outs = Q.quantized_matmul_group(x, [a[0] for a in arrs], [a[1] for a in arrs], mode)
    assert Q.lib.qmm_group_launch_count() == before + 1  # one launch for the group
    check_parts(mode, xb, outs, host, "back to back")
    # the same matrices in another order: still one launch, each result in its slot
    perm = list(reversed(range(len(rows))))
    outs_p = Q.quantized_matmul_group(x, [arrs[i][0] for i in perm], [arrs[i][1] for i in perm], mode)
    assert Q.lib.qmm_group_launch_count() == before + 2
    for j, i in enumerate(perm):
        assert np.array_equal(outs_p[j].numpy(), outs[i].numpy()), (group, i)


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
@pytest.mark.parametrize("M", [1, 3])
def test_group_apart_runs_per_matrix(mode, M):
    """Matrices in separate allocations: one call per matrix, equal to the single calls."""
    import torch

    rows, K = (1000, 37, 530), 5120
    keep, arrs, host = device_group(mode, rows, K, seed=7)
    # copies in separate allocations
    sep = [(Q.Array.from_torch(torch.from_numpy(wq.view(np.int32)).cuda(), dtype=Q.UINT32),
            Q.Array.from_torch(torch.from_numpy(np.ascontiguousarray(s)).cuda())) for wq, s in host]
    xb = bf16(np.random.default_rng(3).standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    before = Q.lib.qmm_group_launch_count()
    outs = Q.quantized_matmul_group(x, [a[0] for a in sep], [a[1] for a in sep], mode)
    assert Q.lib.qmm_group_launch_count() == before
    for (w, s), y in zip(sep, outs):
        assert np.array_equal(y.numpy(), Q.quantized_matmul(x, w, s, mode).numpy())
    check_parts(mode, xb, outs, host, "apart")


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_group_same_kernel_bit_exact(mode, M):
    """Small groups: the one launch (total 1568 rows) and every single call run the
    bf16 GEMV, whose rows do not depend on their neighbours: equal bit for bit."""
    rows, K = (1024, 512, 32), 5120
    keep, arrs, host = device_group(mode, rows, K, seed=11)
    xb = bf16(np.random.default_rng(5).standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    before = Q.lib.qmm_group_launch_count()
    outs = Q.quantized_matmul_group(x, [a[0] for a in arrs], [a[1] for a in arrs], mode)
    assert Q.lib.qmm_group_launch_count() == before + 1
    for (w, s), y in zip(arrs, outs):
        assert np.array_equal(y.numpy(), Q.quantized_matmul(x, w, s, mode).numpy())


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
def test_group_prefill_one_gemm(mode):
    """M > 4: one prefill GEMM over the stacked matrices, each part's columns stored to
    that part; results at the qmm bar."""
    rows, K, M = (256, 64, 32), 512, 40
    keep, arrs, host = device_group(mode, rows, K, seed=13)
    xb = bf16(np.random.default_rng(9).standard_normal((M, K)))
    before = Q.lib.qmm_group_launch_count()
    outs = Q.quantized_matmul_group(Q.Array.from_numpy(xb, Q.BFLOAT16), [a[0] for a in arrs],
                                    [a[1] for a in arrs], mode)
    assert Q.lib.qmm_group_launch_count() == before + 1
    check_parts(mode, xb, outs, host, "prefill")


# The model's groups at prefill sizes: M = 24 and 96 run split tiles (each tile's K over
# several blocks, then the reduce stores to the parts), M = 300 whole tiles with a partial
# last round (mxfp8: 128-tiles in the same launch; nvfp4: 128-row tiles).  Parts whose
# rows are not a multiple of 8 (ragged) take element stores throughout.
@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
@pytest.mark.parametrize("group,M", [("gdn_in_proj", 24), ("gdn_in_proj", 300), ("attn_qkv", 96),
                                     ("attn_qkv", 300), ("ragged_small", 64), ("ragged_big", 200)])
def test_group_prefill_model_shapes(mode, group, M):
    rows, K = GROUPS[group], 5120
    print(f"group {group} {mode} M={M}", flush=True)
    keep, arrs, host = device_group(mode, rows, K, seed=sorted(GROUPS).index(group))
    xb = bf16(np.random.default_rng(100 + M).standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    before = Q.lib.qmm_group_launch_count()
    outs = Q.quantized_matmul_group(x, [a[0] for a in arrs], [a[1] for a in arrs], mode)
    assert Q.lib.qmm_group_launch_count() == before + 1
    # every part at the qmm bar on a row and column sample, against the oracle and against
    # the part's own single call (a different tiling of the same sums)
    rs = np.unique(np.r_[0:M:max(1, M // 7), M - 1])
    for i, (y, (wq, s)) in enumerate(zip(outs, host)):
        n = wq.shape[0]
        cols = np.unique(np.r_[0:n:max(1, n // 300), n - 1])
        yv = y.numpy()
        assert yv.shape == (M, n)
        ref = O.qmm(mode, np.ascontiguousarray(xb[rs]), wq, s, cols=cols)
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(yv[rs][:, cols]), O.bf16_bits_to_f32(ref), **TOL)
        assert ok, (group, i, "oracle", fro, worst)
        single = Q.quantized_matmul(x, arrs[i][0], arrs[i][1], mode).numpy()
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(yv), O.bf16_bits_to_f32(single), **TOL)
        assert ok, (group, i, "single call", fro, worst)
    # a second call gives the same bits (the split tiles' partials are summed in K order)
    outs2 = Q.quantized_matmul_group(x, [a[0] for a in arrs], [a[1] for a in arrs], mode)
    for y, y2 in zip(outs, outs2):
        assert np.array_equal(y.numpy(), y2.numpy())


def test_group_argument_errors():
    keep, arrs, host = device_group("nvfp4", (64, 64), 256, seed=1)
    _, arrs2, _ = device_group("nvfp4", (64,), 512, seed=2)
    x = Q.Array.from_numpy(bf16(np.ones((1, 256))), Q.BFLOAT16)
    with pytest.raises(Q.QmmError, match="K"):
        Q.quantized_matmul_group(x, [arrs[0][0], arrs2[0][0]], [arrs[0][1], arrs2[0][1]], "nvfp4")
    with pytest.raises(Q.QmmError, match="1 to 4"):
        Q.quantized_matmul_group(x, [arrs[0][0]] * 5, [arrs[0][1]] * 5, "nvfp4")


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp8"])
@pytest.mark.parametrize("M", [1, 3])
def test_loader_places_groups_back_to_back(tmp_path, mode, M):
    """A GDN layer's four input projections over two shards: placed back to back
    (weights, and scales), so named_linear_q_group is one launch; a layer missing
    one member keeps separate allocations and runs per matrix."""
    K = 256
    rows = {"in_proj_qkv": 64, "in_proj_z": 32, "in_proj_b": 32, "in_proj_a": 32}
    rng = np.random.default_rng(21)
    q, shard1, shard2 = {}, {}, {}
    for layer in (0, 1):
        pre = f"language_model.model.layers.{layer}.linear_attn."
        for i, (name, n) in enumerate(rows.items()):
            if layer == 1 and name == "in_proj_a":
                continue  # layer 1 lacks a member
            wq, s = O.quantize(mode, O.bf16_bits_to_f32(bf16(rng.standard_normal((n, K)) * 0.05)))
            q[pre + name] = (wq, s)
            dst = shard1 if i % 2 == 0 else shard2
            dst[pre + name + ".weight"] = ("U32", wq)
            dst[pre + name + ".scales"] = ("U8", s)
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors", shard1)
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors", shard2)
    wm = {k: "model-00001-of-00002.safetensors" for k in shard1}
    wm.update({k: "model-00002-of-00002.safetensors" for k in shard2})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    wmap = Q.WeightMap(str(tmp_path))
    xb = bf16(rng.standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    for layer in (0, 1):
        pre = f"language_model.model.layers.{layer}.linear_attn."
        names = [n for n in rows if pre + n in q]
        # bytes unchanged, and placement
        w_ptrs, s_ptrs = [], []
        for n in names:
            w, s = wmap.get(pre + n + ".weight"), wmap.get(pre + n + ".scales")
            assert np.array_equal(w.numpy(), q[pre + n][0]) and np.array_equal(s.numpy(), q[pre + n][1])
            w_ptrs.append((w.ptr, q[pre + n][0].nbytes))
            s_ptrs.append((s.ptr, q[pre + n][1].nbytes))
        adjacent = all(a[0] + a[1] == b[0] for a, b in zip(w_ptrs, w_ptrs[1:])) and \
            all(a[0] + a[1] == b[0] for a, b in zip(s_ptrs, s_ptrs[1:]))
        # layer 0 is placed back to back; layer 1's tensors have allocations of their own
        # (which the allocator could still happen to place adjacently)
        if layer == 0:
            assert adjacent, (w_ptrs, s_ptrs)
        before = Q.lib.qmm_group_launch_count()
        outs = wmap.named_linear_q_group(x, [pre + n + ".weight" for n in names])
        assert Q.lib.qmm_group_launch_count() == before + (1 if adjacent else 0)
        for n, y in zip(names, outs):
            single = wmap.named_linear_q(x, pre + n + ".weight").numpy()
            assert np.array_equal(y.numpy(), single), (layer, n)  # same kernel family at these sizes
            ref = O.qmm(mode, xb, *q[pre + n])
            ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y.numpy()), O.bf16_bits_to_f32(ref), **TOL)
            assert ok, (layer, n, fro, worst)
