"""Writes the golden fixtures in this folder.  Run from the repo root:

    python tests/golden/make_golden.py

reference_qmm_case.json
    The reference's quantized-matmul wiring test (src/model.zig:1561-1609):
    W[o, k] = ((32*o + k) mod 7) - 3 (8 x 32), x[r, k] = ((32*r + k) mod 5) - 2
    (2 x 32), y = x . W^T.  Every group of W has amax 3, so both modes encode
    it exactly; the expected scales, packed words and output follow from the
    format definitions alone, computed here without the oracle:
      * mxfp8: the OCP shared exponent floor(log2 3) - 8 = -7 (E8M0 byte 120);
        elements W / 2^-7 in {-384 .. 384}, encoded by torch's float8_e4m3fn
        cast (an implementation independent of this repository);
      * nvfp4: scale 3 / 6 = 0.5 (E4M3 byte 0x30, again torch's cast); elements
        W / 0.5 in {-6 .. 6}, each exactly an E2M1 value, encoded by table index;
      * packed least significant element first (4 bytes / 8 nibbles per U32);
      * y is the int64 product, exact.

infer_quant_spec_cases.json
    The safetensors headers and expected results of the reference's
    inferQuantSpec test (src/weights.zig:493-541), as data.
"""
import json
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def e4m3_bytes(v):
    return torch.tensor(np.asarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def e2m1_code(v):
    mag = E2M1.index(abs(float(v)))
    return (8 if v < 0 else 0) | mag


def pack(codes, per_word, bits):
    codes = np.asarray(codes, np.uint64)
    n, k = codes.shape
    words = np.zeros((n, k // per_word), np.uint64)
    for j in range(per_word):
        words |= codes[:, j::per_word] << np.uint64(bits * j)
    return words.astype(np.uint32)


def reference_qmm_case():
    W = np.array([(i % 7) - 3 for i in range(8 * 32)], np.int64).reshape(8, 32)
    x = np.array([(i % 5) - 2 for i in range(2 * 32)], np.int64).reshape(2, 32)
    y = x @ W.T
    mx_codes = e4m3_bytes(W * 128.0).reshape(8, 32)  # W / 2^-7
    nv_codes = np.array([[e2m1_code(v / 0.5) for v in row] for row in W], np.uint8)
    nv_scale = int(e4m3_bytes([0.5])[0])
    return {
        "source": "src/model.zig:1561-1609",
        "W": W.tolist(), "x": x.tolist(), "y": y.tolist(),
        "modes": {
            "mxfp8": {"group": 32, "bits": 8, "scales": [[120] * 1] * 8,
                      "w": pack(mx_codes, 4, 8).tolist()},
            "nvfp4": {"group": 16, "bits": 4, "scales": [[nv_scale] * 2] * 8,
                      "w": pack(nv_codes, 8, 4).tolist()},
        },
    }


def infer_quant_spec_cases():
    def hdr(t):
        return json.dumps({k: {"dtype": d, "shape": s, "data_offsets": o} for k, (d, s, o) in t.items()})

    return {
        "source": "src/weights.zig:493-541",
        "cases": [
            {"header": hdr({"l.q_proj.weight": ("U32", [8, 8], [0, 256]),
                            "l.q_proj.scales": ("U8", [8, 4], [256, 288]),
                            "l.norm.weight": ("BF16", [16], [288, 320])}),
             "expect": {"mode": "nvfp4", "group": 16, "bits": 4}},
            {"header": hdr({"l.q_proj.weight": ("U32", [8, 32], [0, 1024]),
                            "l.q_proj.scales": ("U8", [8, 4], [1024, 1056])}),
             "expect": {"mode": "mxfp8", "group": 32, "bits": 8}},
            {"header": hdr({"l.norm.weight": ("BF16", [16], [0, 32])}),
             "expect": {"mode": "none"}},
            {"header": hdr({"l.q_proj.weight": ("U32", [8, 32], [0, 1024]),
                            "l.q_proj.scales": ("BF16", [8, 2], [1024, 1056]),
                            "l.q_proj.biases": ("BF16", [8, 2], [1056, 1088])}),
             "expect": {"error": "AffineUnsupported"}},
            {"header": hdr({"l.q_proj.weight": ("U32", [8, 32], [0, 1024])}),
             "expect": {"error": "NonstandardQuant"}},
        ],
    }


def main():
    (HERE / "reference_qmm_case.json").write_text(json.dumps(reference_qmm_case()) + "\n")
    (HERE / "infer_quant_spec_cases.json").write_text(json.dumps(infer_quant_spec_cases(), indent=1) + "\n")
    print("wrote", HERE / "reference_qmm_case.json", HERE / "infer_quant_spec_cases.json")


if __name__ == "__main__":
    main()
