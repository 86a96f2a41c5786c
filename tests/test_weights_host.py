"""Host-side weight-loading logic through the C ABI, restating the reference's
hermetic tests of src/weights.zig:357-541 (header parse, sanitize, quant-spec
inference).  No GPU work."""
import json

import pytest

import qmm as Q


def test_sanitize_drops_vision_remaps_keeps():
    """src/weights.zig:357-380."""
    assert Q.sanitize_name("vision_tower.blocks.0.attn.proj.weight") is None
    assert Q.sanitize_name("model.visual.proj") is None
    assert Q.sanitize_name("model.language_model.layers.0.q") == "language_model.model.layers.0.q"
    assert Q.sanitize_name("embed_tokens.weight") == "language_model.embed_tokens.weight"
    n = "language_model.model.layers.3.self_attn.q_proj.weight"
    assert Q.sanitize_name(n) == n


def test_header_parse_validates_dtype_and_conv_layout():
    """src/weights.zig:382-404."""
    good = ('{"__metadata__": {}, "a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},\n'
            ' "w": {"dtype": "BF16", "shape": [4, 2], "data_offsets": [8, 24]},\n'
            ' "c": {"dtype": "BF16", "shape": [10240, 4, 1], "data_offsets": [24, 40]}}')
    assert Q.parse_header_json(good) == 3
    assert Q.parse_header_json('{"q": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}}') == "UnsupportedDtype"
    assert Q.parse_header_json(
        '{"m.conv1d.weight": {"dtype": "BF16", "shape": [8, 4, 2], "data_offsets": [0, 128]}}') == "UnsupportedLayout"
    assert Q.parse_header_json(good[:-20]) == "BadHeader"
    assert Q.parse_header_json("not json") == "BadHeader"


def test_infer_quant_spec_reads_mode_group_bits_from_shapes():
    """src/weights.zig:493-541."""
    nv = ('{"l.q_proj.weight": {"dtype": "U32", "shape": [8, 8], "data_offsets": [0, 256]},'
          ' "l.q_proj.scales": {"dtype": "U8", "shape": [8, 4], "data_offsets": [256, 288]},'
          ' "l.norm.weight": {"dtype": "BF16", "shape": [16], "data_offsets": [288, 320]}}')
    assert Q.infer_quant_spec_json(nv) == ("nvfp4", 16, 4)
    mx = ('{"l.q_proj.weight": {"dtype": "U32", "shape": [8, 32], "data_offsets": [0, 1024]},'
          ' "l.q_proj.scales": {"dtype": "U8", "shape": [8, 4], "data_offsets": [1024, 1056]}}')
    assert Q.infer_quant_spec_json(mx) == ("mxfp8", 32, 8)
    dn = '{"l.norm.weight": {"dtype": "BF16", "shape": [16], "data_offsets": [0, 32]}}'
    assert Q.infer_quant_spec_json(dn)[0] == "none"
    aff = ('{"l.q_proj.weight": {"dtype": "U32", "shape": [8, 32], "data_offsets": [0, 1024]},'
           ' "l.q_proj.scales": {"dtype": "BF16", "shape": [8, 2], "data_offsets": [1024, 1056]},'
           ' "l.q_proj.biases": {"dtype": "BF16", "shape": [8, 2], "data_offsets": [1056, 1088]}}')
    assert Q.infer_quant_spec_json(aff) == "AffineUnsupported"
    orph = '{"l.q_proj.weight": {"dtype": "U32", "shape": [8, 32], "data_offsets": [0, 1024]}}'
    assert Q.infer_quant_spec_json(orph) == "NonstandardQuant"


def _hdr(d):
    return json.dumps({k: {"dtype": v[0], "shape": v[1], "data_offsets": [0, 0]} for k, v in d.items()})


@pytest.mark.parametrize("tensors,expect", [
    # second pair disagrees with the first (mxfp8 vs nvfp4 ratio)
    ({"a.weight": ("U32", [8, 32]), "a.scales": ("U8", [8, 4]),
      "b.weight": ("U32", [8, 8]), "b.scales": ("U8", [8, 4])}, "InconsistentQuant"),
    # a second U32 weight with no scales
    ({"a.weight": ("U32", [8, 32]), "a.scales": ("U8", [8, 4]), "b.weight": ("U32", [8, 32])}, "InconsistentQuant"),
    # ratio 4 is neither mode
    ({"a.weight": ("U32", [8, 16]), "a.scales": ("U8", [8, 4])}, "NonstandardQuant"),
    # 3-D scales
    ({"a.weight": ("U32", [8, 32]), "a.scales": ("U8", [8, 4, 1])}, "NonstandardQuant"),
    # scales whose weight is missing
    ({"a.scales": ("U8", [8, 4])}, "NonstandardQuant"),
    # U8 tensor in a dense checkpoint
    ({"a.weight": ("BF16", [8, 32]), "b.idx": ("U8", [4])}, "NonstandardQuant"),
    # a dense bf16 weight beside packed ones is fine (mxfp8 lm_head, src/model.zig:215-216)
    ({"a.weight": ("U32", [8, 32]), "a.scales": ("U8", [8, 4]), "lm_head.weight": ("BF16", [16, 128])},
     ("mxfp8", 32, 8)),
])
def test_infer_quant_spec_rejects_inconsistent_checkpoints(tensors, expect):
    assert Q.infer_quant_spec_json(_hdr(tensors)) == expect


@pytest.mark.parametrize("shape", [[-2, -4], [2147483648, 1], [1, 99999999999999999999], [-1]])
def test_header_rejects_negative_and_oversized_dims(shape):
    """Dimensions must be non-negative and fit an int (the reference's @intCast of a shape
    would fail); two negative dimensions must not pass as a positive element count."""
    h = json.dumps({"w": {"dtype": "U8", "shape": [0], "data_offsets": [0, 8]}}).replace("[0]", json.dumps(shape))
    assert Q.parse_header_json(h) == "BadHeader"
