"""The safetensors -> HBM loader and the named linear dispatch on the GPU.

A small two-shard checkpoint (index json + shards, written here byte by byte in
the safetensors format) holds quantized projections (U32 weights + U8 scales),
a dense BF16 matrix and a norm vector.  The checks follow the reference's
WeightMap.load (src/weights.zig:257-352) and namedLinearQ / linear
(src/model.zig:200-233):
  * tensors come back byte-identical in HBM, at their data_offsets;
  * the quant spec is inferred from the shapes;
  * named_linear_q on a packed weight equals the oracle's qmm of the same bytes,
    and on a dense BF16 weight equals a float64 matmul;
  * a name without ".weight", or a packed weight without scales, is MissingWeight.
"""
import json
import struct

import numpy as np
import pytest

import oracle as O
import qmm as Q

pytestmark = pytest.mark.gpu

TOL = dict(rel_fro=1e-3, ulps=4.0)


def bf16(a):
    return O.f32_to_bf16_bits(np.asarray(a, np.float32))


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, numpy array of the raw element bytes)."""
    header, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def make_checkpoint(tmp_path, mode, N=48, K=256, V=40):
    rng = np.random.default_rng(5 if mode == "mxfp8" else 6)
    pre = "language_model.model.layers.0."
    quant = {}
    for proj in ("mlp.down_proj", "mlp.up_proj"):
        W = O.bf16_bits_to_f32(bf16(rng.standard_normal((N, K)) * 0.02))
        quant[proj] = O.quantize(mode, W)
    dense = bf16(rng.standard_normal((V, K)) * 0.02)
    norm = bf16(rng.standard_normal(K))
    shard1 = {pre + "mlp.down_proj.weight": ("U32", quant["mlp.down_proj"][0]),
              pre + "mlp.down_proj.scales": ("U8", quant["mlp.down_proj"][1]),
              pre + "input_layernorm.weight": ("BF16", norm)}
    shard2 = {pre + "mlp.up_proj.weight": ("U32", quant["mlp.up_proj"][0]),
              pre + "mlp.up_proj.scales": ("U8", quant["mlp.up_proj"][1]),
              "language_model.lm_head.weight": ("BF16", dense)}
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors", shard1)
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors", shard2)
    wm = {k: "model-00001-of-00002.safetensors" for k in shard1}
    wm.update({k: "model-00002-of-00002.safetensors" for k in shard2})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return pre, quant, dense, norm


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
@pytest.mark.parametrize("M", [1, 3, 20])
def test_loader_named_linear_q(tmp_path, mode, M):
    N, K = 48, 256
    pre, quant, dense, norm = make_checkpoint(tmp_path, mode, N=N, K=K)
    wmap = Q.WeightMap(str(tmp_path))
    assert len(wmap) == 6
    assert wmap.quant == (mode, O.GROUP[mode], O.BITS[mode])
    # bytes land unchanged
    wq, s = quant["mlp.up_proj"]
    assert np.array_equal(wmap.get(pre + "mlp.up_proj.weight").numpy(), wq)
    assert np.array_equal(wmap.get(pre + "mlp.up_proj.scales").numpy(), s)
    assert np.array_equal(wmap.get(pre + "input_layernorm.weight").numpy().view(np.uint16), norm)
    rng = np.random.default_rng(M)
    xb = bf16(rng.standard_normal((M, K)))
    x = Q.Array.from_numpy(xb, Q.BFLOAT16)
    for proj in ("mlp.down_proj", "mlp.up_proj"):
        y = wmap.named_linear_q(x, pre + proj + ".weight").numpy()
        ref = O.qmm(mode, xb, *quant[proj])
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(ref), **TOL)
        assert ok, (proj, fro, worst)
    # dense fallback: BF16 weight without scales
    y = wmap.named_linear_q(x, "language_model.lm_head.weight").numpy()
    ref = O.bf16_bits_to_f32(xb).astype(np.float64) @ O.bf16_bits_to_f32(dense).astype(np.float64).T
    refb = np.array([[O.f64_to_bf16_bits(v) for v in r] for r in ref], np.uint16)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(refb), **TOL)
    assert ok, (fro, worst)


def test_loader_missing_weight_errors(tmp_path):
    pre, _, _, _ = make_checkpoint(tmp_path, "nvfp4")
    wmap = Q.WeightMap(str(tmp_path))
    x = Q.Array.from_numpy(bf16(np.ones((1, 256))), Q.BFLOAT16)
    with pytest.raises(Q.QmmError, match="MissingWeight"):
        wmap.named_linear_q(x, pre + "mlp.up_proj")  # no ".weight" suffix
    with pytest.raises(Q.QmmError, match="MissingWeight"):
        wmap.named_linear_q(x, pre + "mlp.gate_proj.weight")  # absent


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
@pytest.mark.parametrize("M", [1, 2])
def test_loader_mtp_names(tmp_path, mode, M):
    """mtpLinearQ (src/mtp.zig:67-70) formats "language_model.mtp.{suffix}" and calls
    namedLinearQ: the MTP head's fc (K = 2 H, src/mtp.zig:158) and its attention
    projections (:85-133) load and dispatch under that prefix like the backbone's."""
    rng = np.random.default_rng(60 + M)
    H = 512
    shapes = {"fc": (H, 2 * H), "layers.0.self_attn.q_proj": (96, H), "layers.0.self_attn.o_proj": (H, 64)}
    q, tensors = {}, {}
    for name, (n, k) in shapes.items():
        q[name] = O.quantize(mode, O.bf16_bits_to_f32(bf16(rng.standard_normal((n, k)) * 0.05)))
        tensors["language_model.mtp." + name + ".weight"] = ("U32", q[name][0])
        tensors["language_model.mtp." + name + ".scales"] = ("U8", q[name][1])
    tensors["language_model.mtp.norm.weight"] = ("BF16", bf16(rng.standard_normal(H)))
    write_safetensors(tmp_path / "model-00001-of-00001.safetensors", tensors)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {k: "model-00001-of-00001.safetensors" for k in tensors}}))
    wmap = Q.WeightMap(str(tmp_path))
    assert wmap.quant == (mode, O.GROUP[mode], O.BITS[mode])
    for name, (n, k) in shapes.items():
        xb = bf16(rng.standard_normal((M, k)))
        y = wmap.named_linear_q(Q.Array.from_numpy(xb, Q.BFLOAT16), "language_model.mtp." + name + ".weight").numpy()
        assert y.shape == (M, n)
        ref = O.qmm(mode, xb, *q[name])
        ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(ref), **TOL)
        assert ok, (name, fro, worst)
    x = Q.Array.from_numpy(bf16(np.ones((1, H))), Q.BFLOAT16)
    with pytest.raises(Q.QmmError, match="MissingWeight"):
        wmap.named_linear_q(x, "language_model.mtp.layers.0.self_attn.k_proj.weight")  # absent
    with pytest.raises(Q.QmmError, match="MissingWeight"):
        wmap.named_linear_q(x, "mtp.fc.weight")  # without the language_model. prefix


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
@pytest.mark.parametrize("M", [1, 20])
def test_loader_mlp_forward_q(tmp_path, mode, M):
    """mlpForwardQ (src/model.zig:905-915): down(silu(gate(x)) * up(x)) by names,
    against the oracle's chain on the same checkpoint bytes."""
    rng = np.random.default_rng(40 + M)
    N, K = 64, 256  # gate / up [N, K], down [K, N]
    pre = "language_model.model.layers.3.mlp."
    q = {}
    for name, (n, k) in (("gate_proj", (N, K)), ("up_proj", (N, K)), ("down_proj", (K, N))):
        q[name] = O.quantize(mode, O.bf16_bits_to_f32(bf16(rng.standard_normal((n, k)) * 0.05)))
    tensors = {}
    for name, (wq, s) in q.items():
        tensors[pre + name + ".weight"] = ("U32", wq)
        tensors[pre + name + ".scales"] = ("U8", s)
    write_safetensors(tmp_path / "model-00001-of-00001.safetensors", tensors)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {k: "model-00001-of-00001.safetensors" for k in tensors}}))
    wmap = Q.WeightMap(str(tmp_path))
    xb = bf16(rng.standard_normal((M, K)))
    y = wmap.mlp_forward_q(Q.Array.from_numpy(xb, Q.BFLOAT16), pre + "gate_proj.weight", pre + "down_proj.weight",
                           pre + "up_proj.weight").numpy()
    h = O.silu_mul_bf16(O.qmm(mode, xb, *q["gate_proj"]), O.qmm(mode, xb, *q["up_proj"]))
    ref = O.qmm(mode, h, *q["down_proj"])
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(ref), **TOL)
    assert ok, (fro, worst)


def test_loader_large_tensors_cycle_the_staging_buffers(tmp_path):
    """A 195.5 MiB packed weight (more than three of the loader's 64 MiB staging chunks,
    so both staging buffers are refilled after their copies were waited for) at an
    unaligned data offset, and its scales with an odd byte count, come back
    byte-identical in HBM (WeightMap.load reads at most 2 GB at a time, AGENTS.md:23)."""
    rng = np.random.default_rng(77)
    N, K = 20001, 16 * 1281  # scales: 20001 x 1281 bytes (odd)
    w = rng.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint32)
    s = rng.integers(0, 256, size=(N, K // 16), dtype=np.uint8)
    norm = bf16(rng.standard_normal(7))
    pre = "language_model.model.layers.0."
    shard = {pre + "input_layernorm.weight": ("BF16", norm), pre + "mlp.down_proj.weight": ("U32", w),
             pre + "mlp.down_proj.scales": ("U8", s)}
    write_safetensors(tmp_path / "model-00001-of-00001.safetensors", shard)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {k: "model-00001-of-00001.safetensors" for k in shard}}))
    assert w.nbytes > 3 * (64 << 20) and s.nbytes % 2 == 1
    wmap = Q.WeightMap(str(tmp_path))
    assert wmap.quant == ("nvfp4", 16, 4)
    assert np.array_equal(wmap.get(pre + "mlp.down_proj.weight").numpy(), w)
    assert np.array_equal(wmap.get(pre + "mlp.down_proj.scales").numpy(), s)
    assert np.array_equal(wmap.get(pre + "input_layernorm.weight").numpy(), norm)
