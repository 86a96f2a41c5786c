"""Pins the CPU oracle (oracle/qmm_oracle.c) before anything is compared with it.

Each check is independent of the oracle's own formula: torch's fp8 dtypes,
closed-form tables, exhaustive brute force, the reference's own test inputs
(src/model.zig:1561-1609) with their closed-form answer, and float64 BLAS.
"""
import numpy as np
import pytest
import torch

import oracle as O


def _same_f32(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(
        np.nan_to_num(a).view(np.uint32), np.nan_to_num(b).view(np.uint32))


# ---------------------------------------------------------------- decoders
def test_e4m3_table_matches_torch_float8_e4m3fn(oracle):
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    assert _same_f32(oracle.e4m3_table(), ref)
    t = oracle.e4m3_table()
    assert t[0x7E] == 448.0 and np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6


def test_e8m0_table_matches_torch_float8_e8m0fnu(oracle):
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e8m0fnu).float().numpy()
    assert _same_f32(oracle.e8m0_table(), ref)
    t = oracle.e8m0_table()
    assert t[127] == 1.0 and t[0] == np.float32(2.0 ** -127) and np.isnan(t[255])


def test_e2m1_table_closed_form_and_e4m3_embedding(oracle):
    t = oracle.e2m1_table()
    mags = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    assert list(t[:8]) == mags
    assert list(-t[8:]) == mags  # sign bit 3 (code 8 is -0)
    assert np.signbit(t[8])
    # Independent pin: nibble (s e1 e0 m) placed as E4M3 byte (s 0 0 e1 e0 m 0 0)
    # decodes (via torch) to e2m1 * 2^-6 for every code.
    emb = torch.tensor([((c & 8) << 4) | ((c & 7) << 2) for c in range(16)], dtype=torch.uint8)
    v = emb.view(torch.float8_e4m3fn).float().numpy() * 64.0
    assert np.array_equal(v, t)


def test_bf16_rounding_matches_torch(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32),
        (rng.standard_normal(1000) * 1e-39).astype(np.float32),  # subnormals
        np.array([3.3895314e38, 3.4e38, -3.4e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 0.0, -0.0], np.float32),
    ])
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.lib().oracle_f32_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(O.f32_to_bf16_bits(vals), ref)
    # one rounding from double: 1 + 2^-8 + 2^-30 rounds up (no double rounding via f32)
    assert oracle.f64_to_bf16_bits(1.0 + 2 ** -8 + 2 ** -30) == 0x3F81


# ---------------------------------------------------------------- packing + dequant
def test_packing_is_lsb_first(oracle):
    w = np.array([[0x76543210]], np.uint32)
    s = np.array([[0x38, 0x38]], np.uint8)  # e4m3 1.0 for nvfp4 groups... K=8 < 16 below
    # nvfp4 row of K=16 (two words), scale 1.0 -> codes 0..7 then 8..15
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    s = np.array([[0x38]], np.uint8)
    d = oracle.dequant("nvfp4", w, s, 16)
    assert np.array_equal(d[0], oracle.e2m1_table())
    # mxfp8 row of K=32: bytes 0..31 in order, scale 2^0
    b = np.arange(32, dtype=np.uint8)
    w = b.view(np.uint32).reshape(1, 8).copy()
    d = oracle.dequant("mxfp8", w, np.array([[127]], np.uint8), 32)
    assert np.array_equal(d[0], oracle.e4m3_table()[:32])


def test_dequant_mxfp8_exhaustive(oracle):
    # row r uses scale byte r for every group; columns cover every code 8x.
    K = 256
    codes = np.arange(256, dtype=np.uint8)
    w = np.tile(codes.view(np.uint32), (256, 1))
    s = np.repeat(np.arange(256, dtype=np.uint8)[:, None], K // 32, axis=1)
    d = oracle.dequant("mxfp8", w, s, K)
    ev = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    sv = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).double().numpy()
    with np.errstate(over="ignore"):
        ref = (sv[:, None] * ev[None, :]).astype(np.float32)
    assert _same_f32(d, ref)
    # invariants: linearity in the scale exponent and sign symmetry
    fin = np.isfinite(d[100]) & np.isfinite(d[101])
    assert np.array_equal(d[101][fin], 2 * d[100][fin])
    assert np.array_equal(d[:, 128:][np.isfinite(d[:, 128:])], -d[:, :128][np.isfinite(d[:, :128])])


def test_dequant_nvfp4_exhaustive(oracle):
    K = 256
    nib = np.arange(16, dtype=np.uint32)
    word = np.uint32(sum(int(c) << (4 * i) for i, c in enumerate(nib[:8])))
    word2 = np.uint32(sum(int(c) << (4 * i) for i, c in enumerate(nib[8:])))
    row = np.tile(np.array([word, word2], np.uint32), K // 16)
    w = np.tile(row, (256, 1))
    s = np.repeat(np.arange(256, dtype=np.uint8)[:, None], K // 16, axis=1)
    d = oracle.dequant("nvfp4", w, s, K)
    sv = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    ev = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    ref = (sv[:, None] * np.tile(ev, K // 16)[None, :]).astype(np.float32)
    assert _same_f32(d, ref)
    # zero scale -> 0; every finite value exact in bf16 (e2m1 * e4m3 <= 6 significant bits)
    assert np.all(d[0] == 0)
    fin = d[np.isfinite(d)]
    assert np.array_equal(O.bf16_bits_to_f32(O.f32_to_bf16_bits(fin)), fin)


def test_dequant_bf16_is_rounded_f32(oracle):
    rng = np.random.default_rng(3)
    for mode in ("mxfp8", "nvfp4"):
        K = 128
        w = rng.integers(0, 2 ** 32, size=(16, K * O.BITS[mode] // 32), dtype=np.uint32)
        s = rng.integers(100, 140, size=(16, K // O.GROUP[mode]), dtype=np.uint8)
        f = oracle.dequant(mode, w, s, K)
        b = oracle.dequant_bf16(mode, w, s, K)
        assert np.array_equal(b, O.f32_to_bf16_bits(f))


# ---------------------------------------------------------------- quantize
def _brute_quantize(mode, W):
    """Independent brute-force restatement of the documented quantizer rule."""
    e4 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    pos = np.arange(0x7F)  # finite non-negative e4m3 codes 0..0x7E
    N, K = W.shape
    g = O.GROUP[mode]
    codes = np.zeros((N, K), np.uint32)
    scales = np.zeros((N, K // g), np.uint8)
    e2 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6])
    for n in range(N):
        for gi in range(K // g):
            v = W[n, gi * g:(gi + 1) * g].astype(np.float64)
            amax = np.max(np.abs(v))
            if mode == "mxfp8":
                X = 0 if amax == 0 else int(np.clip(np.floor(np.log2(amax)) - 8 + 127, 0, 254))
                sc = 2.0 ** (X - 127)
                scales[n, gi] = X
                cand = e4[pos] * sc
                for i, x in enumerate(v):
                    d = np.abs(cand - abs(x))
                    best = np.flatnonzero(d == d.min())
                    c = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
                    if np.signbit(x) and c != 0:
                        c |= 0x80
                    codes[n, gi * g + i] = c
            else:
                d = np.abs(6.0 * e4[pos] - amax)
                best = np.flatnonzero(d == d.min())
                sc_code = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
                scales[n, gi] = sc_code
                sc = e4[sc_code]
                for i, x in enumerate(v):
                    if sc == 0:
                        c = 0
                    else:
                        dd = np.abs(e2 * sc - abs(x))
                        best = np.flatnonzero(dd == dd.min())
                        c = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
                        if np.signbit(x) and c != 0:
                            c |= 0x8
                    codes[n, gi * g + i] = c
    return codes, scales


def _pack(mode, codes):
    N, K = codes.shape
    if mode == "mxfp8":
        return codes.astype(np.uint8).reshape(N, K // 4, 4).view(np.uint32).reshape(N, K // 4)
    c = codes.reshape(N, K // 8, 8).astype(np.uint32)
    return np.bitwise_or.reduce(c << (4 * np.arange(8, dtype=np.uint32)), axis=2)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_quantize_matches_brute_force(oracle, mode):
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((6, 128)) * 0.02).astype(np.float32)
    W = O.bf16_bits_to_f32(O.f32_to_bf16_bits(W))  # bf16-valued, like the configs
    W[0, :32] = 0.0  # an all-zero group
    W[1, 5] = 1e4  # saturating group
    # exact tie cases for nvfp4 (scale 1.0 group: amax 6): 0.25, 0.75, 2.5, 5.0
    W[2, 64:80] = [6, .25, .75, 1.25, 1.75, 2.5, 3.5, 5, -.25, -.75, -2.5, -5, 0, 1, 2, 3]
    wq, s = oracle.quantize(mode, W)
    codes, sc = _brute_quantize(mode, W)
    assert np.array_equal(s, sc)
    assert np.array_equal(wq, _pack(mode, codes))


def test_e4m3_encode_matches_torch_cast(oracle):
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(3000) * 50, rng.standard_normal(1000) * 0.01,
                        [448.0, -448.0, 2 ** -9, 2 ** -10, 3 * 2 ** -11, 0.0]])
    v = v[np.abs(v) <= 448]  # torch does not saturate above 448
    v32 = v.astype(np.float32)
    ref = torch.from_numpy(v32).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.lib().oracle_e4m3_encode(float(x)) for x in v32], np.uint8)
    # torch maps -0.0 / tiny negatives to 0x80; the oracle writes +0 for a zero code
    ref = np.where(ref == 0x80, 0, ref)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- the reference test, restated
def _ref_test_inputs():
    # src/model.zig:1567-1570: W[o,k] = ((o*32+k) mod 7) - 3 (8x32), x[r,k] = ((r*32+k) mod 5) - 2 (2x32)
    W = np.array([(i % 7) - 3 for i in range(8 * 32)], np.float32).reshape(8, 32)
    x = np.array([(i % 5) - 2 for i in range(2 * 32)], np.float32).reshape(2, 32)
    return W, x


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_reference_qmm_case_is_exact(oracle, mode):
    W, x = _ref_test_inputs()
    wq, s = oracle.quantize(mode, W)
    # closed form: every group has amax 3 -> mxfp8 scale 2^-7 (byte 120), nvfp4 scale 0.5 (0x30)
    assert np.all(s == (120 if mode == "mxfp8" else 0x30))
    assert np.array_equal(oracle.dequant(mode, wq, s, 32), W)
    yexp = (x.astype(np.int64) @ W.astype(np.int64).T).astype(np.float32)
    for xin, isbf in ((O.f32_to_bf16_bits(x), True), (x, False)):
        y = oracle.qmm(mode, xin, wq, s, x_is_bf16=isbf, out="f32")
        assert np.array_equal(y, yexp)
    yb = oracle.qmm(mode, O.f32_to_bf16_bits(x), wq, s)
    assert np.array_equal(O.bf16_bits_to_f32(yb), yexp)


# ---------------------------------------------------------------- qmm vs float64 BLAS
@pytest.mark.parametrize("mode,M,N,K", [("mxfp8", 3, 96, 256), ("nvfp4", 4, 80, 512), ("nvfp4", 1, 33, 48)])
def test_qmm_matches_float64_blas(oracle, mode, M, N, K):
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, s = oracle.quantize(mode, W)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    # independent dequant through torch's fp8 tables
    e4 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    e8 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).double().numpy()
    e2 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    if mode == "mxfp8":
        c = wq.view(np.uint8).reshape(N, K)
        D = e4[c] * np.repeat(e8[s], 32, axis=1)
    else:
        c = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K)
        D = e2[c] * np.repeat(e4[s], 16, axis=1)
    ref = O.bf16_bits_to_f32(xb).astype(np.float64) @ D.T
    refb = np.array([[O.f64_to_bf16_bits(v) for v in row] for row in ref], np.uint16)
    y = oracle.qmm(mode, xb, wq, s)
    assert np.array_equal(y, refb)
    # column subset returns the same values
    cols = np.array([N - 1, 0, N // 2], np.int64)
    assert np.array_equal(oracle.qmm(mode, xb, wq, s, cols=cols), refb[:, cols])
    # fp32-accumulating CPU-baseline form stays inside the north-star bound
    y32 = oracle.qmm(mode, xb, wq, s, f32acc=True)
    ok, fro, worst = O.check_tolerance(O.bf16_bits_to_f32(y32), O.bf16_bits_to_f32(refb))
    assert ok, (fro, worst)


def test_qmm_special_weights_closed_forms(oracle):
    """The special-value semantics of the parity oracle, each case a closed form: an
    mxfp8 weight 448 * 2^(X-127) whose f32 dequant overflows multiplies x exactly
    (x = 2^-10 gives 1.75 * 2^(X-129); x = 0 gives 0); x = +-1.5 against it overflows
    to +-inf from X = 247; a NaN scale or NaN element code makes the output NaN even against x = 0;
    nvfp4 scale 0x01 (2^-9) and 0 are exact, 0x7F / 0xFF are NaN."""
    K = 64
    for X in (240, 247, 254):
        codes = np.zeros(K, np.uint8)
        codes[5] = 0x7E
        wq = codes.view(np.uint32).reshape(1, K // 4)
        s = np.full((1, K // 32), X, np.uint8)
        assert np.isinf(oracle.dequant("mxfp8", wq, s, K)[0, 5]) == (X >= 247)
        x = np.zeros((4, K), np.float32)
        x[0, 5], x[1, 5], x[2, 5], x[3, 5] = 2.0 ** -10, 0.0, 1.5, -1.5
        y = O.bf16_bits_to_f32(oracle.qmm("mxfp8", O.f32_to_bf16_bits(x), wq, s)).astype(np.float64)
        assert y[0, 0] == 1.75 * 2.0 ** (X - 129) and y[1, 0] == 0.0
        big = np.inf if X >= 247 else 1.5 * 448.0 * 2.0 ** (X - 127)  # exact in bf16 below overflow
        assert y[2, 0] == big and y[3, 0] == -big
    x = O.f32_to_bf16_bits(np.zeros((1, K), np.float32))
    for code, sb in ((0x7F, 127), (0xFF, 127), (0x00, 0xFF)):
        codes = np.zeros(K, np.uint8)
        codes[40] = code
        y = oracle.qmm("mxfp8", x, codes.view(np.uint32).reshape(1, K // 4), np.array([[127, sb]], np.uint8))
        assert np.isnan(O.bf16_bits_to_f32(y)).all(), (code, sb)
    nib = np.zeros((1, K // 8), np.uint32)
    nib[0, 0] = 0x7  # element 0 = 6.0
    xo = np.zeros((1, K), np.float32)
    xo[0, 0] = 1.0
    for sb, want in ((0x01, 6.0 * 2.0 ** -9), (0x00, 0.0), (0x7F, np.nan), (0xFF, np.nan)):
        s = np.full((1, K // 16), 0x38, np.uint8)
        s[0, 0] = sb
        y = O.bf16_bits_to_f32(oracle.qmm("nvfp4", O.f32_to_bf16_bits(xo), nib, s))[0, 0]
        assert (np.isnan(y) and np.isnan(want)) or y == want, (sb, y)


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_qmm_special_weights_match_torch_tables(oracle, mode):
    """Every scale byte (NaN included) and every element code (NaN codes included) on random
    rows, against an independent product: torch's float8_e4m3fn / float8_e8m0fnu tables in
    float64 (exact products, no f32 dequant), a float64 matmul, one rounding to bf16."""
    rng = np.random.default_rng(31)
    N, K, M = 512, 256, 3
    g = 32 if mode == "mxfp8" else 16
    e4 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    e8 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).double().numpy()
    e2 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    if mode == "mxfp8":
        c = rng.integers(0, 256, size=(N, K), dtype=np.uint8)
        c[: N // 2] &= 0xF7  # no NaN code in the first half (S.1111.111 needs bit 3)
        s = np.repeat(rng.integers(0, 256, size=(N, 1), dtype=np.uint8), K // g, axis=1)
        s[: N // 2] = np.arange(N // 2)[:, None] % 255  # every non-NaN byte, one per row
        wq = np.ascontiguousarray(c).view(np.uint32).reshape(N, K // 4)
        D = e4[c] * np.repeat(e8[s], g, axis=1)
    else:
        c = rng.integers(0, 16, size=(N, K), dtype=np.uint32)
        s = rng.integers(0, 256, size=(N, K // g), dtype=np.uint8)
        s[: N // 2] = (np.arange(N // 2)[:, None] + np.arange(K // g)[None, :]) % 127
        wq = np.zeros((N, K // 8), np.uint32)
        for i in range(8):
            wq |= c[:, i::8] << np.uint32(4 * i)
        D = e2[c] * np.repeat(e4[s], g, axis=1)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = O.bf16_bits_to_f32(xb).astype(np.float64) @ D.T
    y = O.bf16_bits_to_f32(oracle.qmm(mode, xb, wq, s)).astype(np.float64)
    assert np.isnan(ref).any() and np.isfinite(ref).any()
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(y[fin], O.bf16_bits_to_f32(O.f64_to_bf16_bits_vec(ref[fin])).astype(np.float64))
    assert np.array_equal(y[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])


def test_tolerance_rejects_planted_mistakes(oracle):
    """A transposed operand, a dropped scale or a wrong group index must fail the bound."""
    rng = np.random.default_rng(9)
    mode, M, N, K = "nvfp4", 2, 64, 256
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, s = oracle.quantize(mode, W)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    good = O.bf16_bits_to_f32(oracle.qmm(mode, xb, wq, s))
    # dropped per-group scale variation (all scales forced to the row's first)
    s_bad = np.repeat(s[:, :1], s.shape[1], axis=1)
    bad1 = O.bf16_bits_to_f32(oracle.qmm(mode, xb, wq, s_bad))
    # scale index off by one group
    bad2 = O.bf16_bits_to_f32(oracle.qmm(mode, xb, wq, np.roll(s, 1, axis=1)))
    # nibble order reversed inside each word
    rev = np.zeros_like(wq)
    for i in range(8):
        rev |= ((wq >> (4 * i)) & 0xF) << (4 * (7 - i))
    bad3 = O.bf16_bits_to_f32(oracle.qmm(mode, xb, rev, s))
    for bad in (bad1, bad2, bad3):
        ok, _, _ = O.check_tolerance(bad, good)
        assert not ok
    ok, fro, worst = O.check_tolerance(good, good)
    assert ok and fro == 0 and worst == 0


# ---------------------------------------------------------------- MLP activation
def test_f64_to_bf16_vec_matches_scalar(oracle):
    rng = np.random.default_rng(21)
    v = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-40, 38, 2000),
                        [0.0, -0.0, 1e-45, -3e-39, 3.4e38, -3.39e38, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9]])
    got = O.f64_to_bf16_bits_vec(v)
    ref = np.array([O.f64_to_bf16_bits(x) for x in v], np.uint16)
    assert np.array_equal(got, ref)


def test_silu_mul_matches_torch_bf16_ops():
    """The oracle's op-by-op bf16 chain against torch's CPU bf16 ops (sigmoid, two
    multiplies, each rounding to bf16).  torch evaluates sigmoid in float32, the
    oracle in float64: they may differ by one bf16 ulp where the two straddle a
    rounding boundary."""
    rng = np.random.default_rng(22)
    g = O.f32_to_bf16_bits(rng.standard_normal(20000).astype(np.float32) * 4)
    u = O.f32_to_bf16_bits(rng.standard_normal(20000).astype(np.float32))
    got = O.silu_mul_bf16(g, u)
    gt = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    ut = torch.from_numpy(u.view(np.int16)).view(torch.bfloat16)
    ref = ((gt * torch.sigmoid(gt)) * ut).view(torch.int16).numpy().view(np.uint16)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999
    # closed forms: silu(0) = 0, large positive g -> g * u, large negative -> 0
    z = O.f32_to_bf16_bits(np.array([0.0, 100.0, -100.0], np.float32))
    one = O.f32_to_bf16_bits(np.array([3.0, 2.0, 5.0], np.float32))
    assert np.array_equal(O.bf16_bits_to_f32(O.silu_mul_bf16(z, one)), np.array([0.0, 200.0, -0.0], np.float32))
