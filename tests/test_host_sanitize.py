"""The checkpoint parser (mlx-runner_amd/csrc/checkpoint.cpp: parseHeaderJson,
inferQuantSpec, sanitizeName and the index / shard-header half of WeightMap.load,
src/weights.zig:70-300) built for the host with AddressSanitizer and
UndefinedBehaviorSanitizer (g++, no GPU), and run over

  * the reference's header cases (src/weights.zig:382-404, :493-541),
  * seeded mutations of them (byte flips, truncations, inserted tokens such as
    huge or negative numbers), and
  * checkpoint directories with corrupt headers: negative dimensions, dimensions
    above INT32_MAX, a byte count that overflows 64 bits, offsets that disagree
    with the shape, header lengths past the file, missing shards, a broken index,
    duplicate names, too many dimensions.

Any sanitizer report aborts the driver (non-zero exit); every return code must be
0 or a loader error code.
"""
import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
WE = {"BadIndexJson": 101, "BadHeader": 102, "UnsupportedDtype": 103, "UnsupportedLayout": 104,
      "DuplicateTensor": 106, "NonstandardQuant": 107, "InconsistentQuant": 108, "AffineUnsupported": 109, "IO": 110}


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not found")
    out = tmp_path_factory.mktemp("san") / "checkpoint_fuzz"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", str(ROOT / "include"), str(ROOT / "mlx-runner_amd/csrc/checkpoint.cpp"),
           str(HERE / "host_sanitize/checkpoint_fuzz.cpp"), "-o", str(out)]
    subprocess.run(cmd, check=True, timeout=600)
    return out


def run(driver, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(driver), *map(str, args)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-4000:])
    return r.stdout


def reference_headers():
    cases = json.loads((HERE / "golden/infer_quant_spec_cases.json").read_text())["cases"]
    out = [(c["header"], 0 if "mode" in c["expect"] else WE[c["expect"]["error"]]) for c in cases]
    out += [
        ('{"__metadata__": {}, "a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},\n'
         ' "w": {"dtype": "BF16", "shape": [4, 2], "data_offsets": [8, 24]},\n'
         ' "c": {"dtype": "BF16", "shape": [10240, 4, 1], "data_offsets": [24, 40]}}', 0),
        ('{"q": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}}', WE["UnsupportedDtype"]),
        ('{"m.conv1d.weight": {"dtype": "BF16", "shape": [8, 4, 2], "data_offsets": [0, 128]}}',
         WE["UnsupportedLayout"]),
        ('{"w": {"dtype": "U8", "shape": [-2, -4], "data_offsets": [0, 8]}}', WE["BadHeader"]),
        ('{"w": {"dtype": "U8", "shape": [2147483648, 1], "data_offsets": [0, 8]}}', WE["BadHeader"]),
        ('{"w": {"dtype": "U8", "shape": [99999999999999999999], "data_offsets": [0, 8]}}', WE["BadHeader"]),
    ]
    return out


def test_reference_headers_under_sanitizers(driver, tmp_path):
    files = []
    for i, (h, want) in enumerate(reference_headers()):
        p = tmp_path / f"h{i}.json"
        p.write_text(h)
        files.append((p, want))
    out = run(driver, "header", *[p for p, _ in files]).splitlines()
    for (p, want), line in zip(files, out):
        assert line == f"{p} rc={want}", (line, want)


def test_mutated_headers_under_sanitizers(driver, tmp_path):
    files = []
    for i, (h, _) in enumerate(reference_headers()[:6]):
        p = tmp_path / f"m{i}.json"
        p.write_text(h)
        files.append(p)
    out = run(driver, "mutate", 3000, *files)
    assert out.count("mutations=3000") == len(files), out


def write_checkpoint(d: Path, shards: dict, index: dict | None = None, raw_len: dict | None = None):
    """shards: file name -> {tensor: (dtype, shape, (off0, off1))}; data is zeros of the
    largest end offset.  raw_len: file name -> header length field to write instead."""
    d.mkdir()
    wm = {}
    for fname, tensors in shards.items():
        hdr = json.dumps({k: {"dtype": v[0], "shape": v[1], "data_offsets": list(v[2])} for k, v in tensors.items()})
        hb = hdr.encode()
        end = max([v[2][1] for v in tensors.values() if v[2][1] < (1 << 20)] + [0])
        n = (raw_len or {}).get(fname, len(hb))
        (d / fname).write_bytes(struct.pack("<Q", n) + hb + bytes(end))
        for k in tensors:
            wm[k] = fname
    (d / "model.safetensors.index.json").write_text(json.dumps(index if index is not None else {"weight_map": wm}))


def test_checkpoint_directories_under_sanitizers(driver, tmp_path):
    U32, U8 = "U32", "U8"
    good = {"a.safetensors": {"l.q_proj.weight": (U32, [8, 8], (0, 256)), "l.q_proj.scales": (U8, [8, 4], (256, 288))},
            "b.safetensors": {"l.norm.weight": ("BF16", [16], (0, 32))}}
    cases = {
        "good": (dict(shards=good), "rc=0 tensors=3"),
        "negative_dims": (dict(shards={"a.safetensors": {"w": (U8, [-2, -4], (0, 8))}}), f"rc={WE['BadHeader']}"),
        "dim_over_int32": (dict(shards={"a.safetensors": {"w": (U8, [2147483648], (0, 8))}}), f"rc={WE['BadHeader']}"),
        "bytes_overflow": (dict(shards={"a.safetensors": {"w": (U32, [2147483647] * 4, (0, 4))}}),
                           f"rc={WE['BadHeader']}"),
        "offsets_disagree": (dict(shards={"a.safetensors": {"w": (U32, [8, 8], (0, 255))}}), f"rc={WE['BadHeader']}"),
        "negative_offset": (dict(shards={"a.safetensors": {"w": (U8, [4], (-4, 0))}}), f"rc={WE['BadHeader']}"),
        "nine_dims": (dict(shards={"a.safetensors": {"w": (U8, [1] * 9, (0, 1))}}), f"rc={WE['BadHeader']}"),
        "header_len_huge": (dict(shards=good, raw_len={"a.safetensors": 1 << 40}), f"rc={WE['BadHeader']}"),
        "header_len_past_eof": (dict(shards=good, raw_len={"b.safetensors": 1 << 20}), f"rc={WE['IO']}"),
        "header_len_zero": (dict(shards=good, raw_len={"a.safetensors": 0}), f"rc={WE['BadHeader']}"),
        "missing_shard": (dict(shards=good, index={"weight_map": {"x.weight": "nope.safetensors"}}), f"rc={WE['IO']}"),
        "bad_index": (dict(shards=good, index={"weight_map": ["a.safetensors"]}), f"rc={WE['BadIndexJson']}"),
        "duplicate": (dict(shards={"a.safetensors": {"l.w": (U8, [4], (0, 4))},
                                   "b.safetensors": {"language_model.l.w": (U8, [4], (0, 4))}}),
                      f"rc={WE['DuplicateTensor']}"),
    }
    dirs = []
    for name, (kw, _) in cases.items():
        write_checkpoint(tmp_path / name, **kw)
        dirs.append(tmp_path / name)
    out = run(driver, "dir", *dirs).splitlines()
    for (name, (_, want)), line in zip(cases.items(), out):
        assert line.startswith(str(tmp_path / name) + " " + want), (name, line, want)
