"""Special and extreme weight values through every quantized-matmul kernel family.

The reference computes x @ deq(W).T over mlx_dequantize (src/model.zig:1589-1593).
What it does with NaN codes, NaN scales and weights whose f32 dequant overflows
is MLX's (not importable here), so the semantics are this library's, stated in
the oracle: a weight is elem * scale taken exactly, a NaN element code (E4M3
S.1111.111) or NaN scale (E8M0 0xFF; E4M3 S.1111.111) makes it NaN, and y is
the sum rounded once to bf16 (overflow to +-inf).

Weight rows come in classes (row n, class n % 16):
  mxfp8  0-9   every group's E8M0 scale byte (37 n) % 247 (0..246: 2^-127 .. 2^119),
               random non-NaN E4M3 codes, small ones above byte 200 (no overflow)
         10    as 0-9 with one group's scale byte 0xFF (NaN)      -> y NaN
         11    as 0-9 with one element code 0x7F or 0xFF (NaN)    -> y NaN
         12    scale bytes 247-254, one code +-448 at k0 (x = +-1.5 there) -> y +-inf
         13    scale bytes 240-254, one code 448 at k1 (x = 2^-10 there): the f32
               dequant of that weight overflows, the product does not -> y finite, exact
         14    scale byte 254, one code 448 at k2 (x = 0 there)   -> y = 0
         15    random scale bytes 100-154 per group, random codes
  nvfp4  0-9   every group's E4M3 scale byte (37 n) % 127 (0x00..0x7E: zero, subnormals,
               up to 448), random E2M1 codes
         10    one group's scale byte 0x7F (NaN)                  -> y NaN
         11    one group's scale byte 0xFF (NaN)                  -> y NaN
         12-15 random scale bytes 0x00-0x7E per group, random codes
x is N(0,1) bf16 with x[:, k0] = +-1.5, x[:, k1] = 2^-10 and x[:, k2] = 0.

Bar: NaN and +-inf positions (and signs) equal the oracle's; every finite output
within 4 bf16 ulps of its own scale, max(|y|, sqrt(sum_k (x_k w_k)^2)) (rows of y
here span 2^250, so "the row's output scale" is taken per output).
"""
import numpy as np
import pytest

import oracle as O
import qmm as Q

pytestmark = pytest.mark.gpu

E4M3_NAN = (0x7F, 0xFF)


def _codes_mxfp8(rng, shape, small):
    """Random non-NaN E4M3 codes; `small`: magnitudes below 0.25 (exponent field <= 4)."""
    mag = rng.integers(0, 0x28 if small else 0x7F, size=shape, dtype=np.uint8)
    return mag | (rng.integers(0, 2, size=shape, dtype=np.uint8) << 7)


def special_weights(mode, N, K, seed):
    """(packed u32 [N, K*bits/32], scales u8 [N, K/group], (k0, k1, k2))."""
    rng = np.random.default_rng(seed)
    g = 32 if mode == "mxfp8" else 16
    G = K // g
    k0, k1, k2 = 37 % K, (K // 2 + 70) % K, K - 9
    n = np.arange(N)
    cls = n % 16
    if mode == "mxfp8":
        sweep = ((37 * n) % 247).astype(np.uint8)
        s = np.repeat(sweep[:, None], G, axis=1)
        codes = np.zeros((N, K), np.uint8)
        for small in (False, True):
            rows = (cls <= 11) & ((sweep > 200) == small)
            codes[rows] = _codes_mxfp8(rng, (int(rows.sum()), K), small)
        r10 = np.nonzero(cls == 10)[0]
        s[r10, rng.integers(0, G, size=r10.size)] = 0xFF
        r11 = np.nonzero(cls == 11)[0]
        codes[r11, rng.integers(0, K, size=r11.size)] = rng.choice(E4M3_NAN, size=r11.size)
        r12 = np.nonzero(cls == 12)[0]
        s[r12] = (247 + (r12 // 16) % 8)[:, None]
        codes[r12, k0] = np.where((r12 // 16) % 2 == 0, 0x7E, 0xFE)
        r13 = np.nonzero(cls == 13)[0]
        s[r13] = (240 + (r13 // 16) % 15)[:, None]
        codes[r13, k1] = 0x7E
        r14 = np.nonzero(cls == 14)[0]
        s[r14] = 254
        codes[r14, k2] = 0x7E
        r15 = np.nonzero(cls == 15)[0]
        s[r15] = rng.integers(100, 155, size=(r15.size, G), dtype=np.uint8)
        codes[r15] = _codes_mxfp8(rng, (r15.size, K), False)
        wq = np.ascontiguousarray(codes).view(np.uint32).reshape(N, K // 4)
    else:
        sweep = ((37 * n) % 127).astype(np.uint8)
        s = np.repeat(sweep[:, None], G, axis=1)
        r10 = np.nonzero(cls == 10)[0]
        s[r10, rng.integers(0, G, size=r10.size)] = 0x7F
        r11 = np.nonzero(cls == 11)[0]
        s[r11, rng.integers(0, G, size=r11.size)] = 0xFF
        rmix = np.nonzero(cls >= 12)[0]
        s[rmix] = rng.integers(0, 0x7F, size=(rmix.size, G), dtype=np.uint8)
        nib = rng.integers(0, 16, size=(N, K), dtype=np.uint32)
        wq = np.zeros((N, K // 8), np.uint32)
        for i in range(8):
            wq |= nib[:, i::8] << np.uint32(4 * i)
    return np.ascontiguousarray(wq), np.ascontiguousarray(s), (k0, k1, k2)


def special_x(M, K, ks, seed, f32=False):
    k0, k1, k2 = ks
    x = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)
    x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))
    x[:, k0] = np.where(np.arange(M) % 2 == 0, 1.5, -1.5)
    x[:, k1] = 2.0 ** -10
    x[:, k2] = 0.0
    return x if f32 else O.f32_to_bf16_bits(x)


def output_scale(mode, x, wq, s, K):
    """max(|y_ref|, sqrt(sum_k (x_k w_k)^2)) per output, with exact weights (float64)."""
    xd = np.asarray(x, np.float64) ** 2
    N = wq.shape[0]
    out = np.empty((x.shape[0], N))
    for r0 in range(0, N, 512):
        D = O.dequant_f64(mode, wq[r0:r0 + 512], s[r0:r0 + 512], K)
        with np.errstate(invalid="ignore", over="ignore"):
            out[:, r0:r0 + 512] = np.sqrt(xd @ (D * D).T)
    return out


def check_special(mode, got, ref, xval, wq, s, K):
    """NaN / inf positions equal, finite values within 4 ulps of each output's scale."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(r)), np.argwhere(np.isnan(g) != np.isnan(r))[:8]
    assert np.array_equal(np.isposinf(g), np.isposinf(r)), np.argwhere(np.isposinf(g) != np.isposinf(r))[:8]
    assert np.array_equal(np.isneginf(g), np.isneginf(r)), np.argwhere(np.isneginf(g) != np.isneginf(r))[:8]
    fin = np.isfinite(r)
    scale = np.maximum(output_scale(mode, xval, wq, s, K), np.abs(r))
    ulp = np.maximum(2.0 ** (np.floor(np.log2(np.where(scale > 0, scale, 1.0))) - 7), 2.0 ** -133)
    with np.errstate(invalid="ignore"):
        err = np.where(fin, np.abs(g - r), 0.0)
    worst = np.max(err / ulp)
    bad = np.argwhere(err > 4 * ulp)
    assert worst <= 4.0, (worst, bad[:8], [(g[tuple(b)], r[tuple(b)]) for b in bad[:4]])
    return worst


# (mode, M, N, K, x form): one shape per kernel family run_qmm selects (bf16 x unless noted)
FAMILIES = [
    ("mxfp8", 1, 1024, 5120, "bf16"),     # unpacking GEMV, one segment per row
    ("mxfp8", 1, 1024, 17408, "bf16"),    # long-row unpacking GEMV
    ("mxfp8", 2, 4096, 5120, "bf16"),     # scaled-MFMA GEMV 16x16x128, one pass
    ("mxfp8", 4, 4096, 17408, "bf16"),    # scaled-MFMA GEMV, three passes
    ("mxfp8", 6, 1024, 5120, "bf16"),     # unpacking GEMV, M = 6
    ("mxfp8", 300, 1000, 1024, "bf16"),   # prefill GEMM on the scaled fp8 MFMA (pipelined)
    ("mxfp8", 300, 1000, 1056, "bf16"),   # prefill GEMM, K not a multiple of 128
    ("mxfp8", 2, 512, 1024, "f32"),       # f32 x GEMV
    ("mxfp8", 2, 512, 1024, "unaligned"),  # any-shape GEMV (x not 16-byte aligned)
    ("nvfp4", 1, 1024, 5120, "bf16"),     # unpacking GEMV
    ("nvfp4", 1, 16400, 5120, "bf16"),    # scaled-MFMA GEMV 16x16x128, M = 1
    ("nvfp4", 1, 5120, 17408, "bf16"),    # scaled-MFMA GEMV, three passes
    ("nvfp4", 2, 4099, 5120, "bf16"),     # scaled-MFMA GEMV, M = 2
    ("nvfp4", 3, 4099, 5120, "bf16"),     # 32x32x64 MFMA GEMV, one pass
    ("nvfp4", 3, 5120, 17408, "bf16"),    # 32x32x64 MFMA GEMV, several passes
    ("nvfp4", 6, 512, 5120, "bf16"),      # unpacking GEMV, M = 6
    ("nvfp4", 6, 4099, 5120, "bf16"),     # dequantizing bf16-MFMA GEMV, x of 5-8 rows
    ("nvfp4", 12, 4099, 5120, "bf16"),    # the same, x of 9-16 rows
    ("nvfp4", 16, 1024, 6144, "bf16"),    # the same at K = 6144 (12 waves)
    ("nvfp4", 300, 1000, 1024, "bf16"),   # prefill GEMM on the bf16 MFMA
    ("nvfp4", 2, 512, 1024, "f32"),       # f32 x GEMV
    ("nvfp4", 2, 64, 48, "bf16"),         # any-shape GEMV (24-byte rows)
    ("nvfp4", 2, 512, 1024, "unaligned"),  # any-shape GEMV (x not 16-byte aligned)
]


@pytest.mark.parametrize("mode,M,N,K,xform", FAMILIES)
def test_special_weights_every_kernel_family(mode, M, N, K, xform):
    seed = 1000 + 7 * M + N % 97 + K % 89
    wq, s, ks = special_weights(mode, N, K, seed)
    f32 = xform == "f32"
    x = special_x(M, K, ks, seed + 1, f32=f32)
    xval = x if f32 else O.bf16_bits_to_f32(x)
    if xform == "unaligned":
        import torch

        flat = torch.from_numpy(x.view(np.int16).reshape(-1).copy())
        buf = torch.empty(M * K + 8, dtype=torch.int16, device="cuda")
        buf[1:1 + M * K] = flat.cuda()
        xt = buf[1:1 + M * K].view(torch.bfloat16).view(M, K)
        assert xt.data_ptr() % 16 != 0
        xa = Q.Array.from_torch(xt)
    else:
        xa = Q.Array.from_numpy(x, Q.FLOAT32 if f32 else Q.BFLOAT16)
    y = Q.quantized_matmul(xa, Q.Array.from_numpy(wq, Q.UINT32), Q.Array.from_numpy(s, Q.UINT8), mode).numpy()
    if f32:
        ref = O.qmm(mode, x, wq, s, x_is_bf16=False, out="f32")
        got = y
    else:
        ref = O.bf16_bits_to_f32(O.qmm(mode, x, wq, s))
        got = O.bf16_bits_to_f32(y)
    # the construction's promises hold in the oracle: each class gives what it says
    cls = np.arange(N) % 16
    if mode == "mxfp8":
        assert np.isnan(ref[:, cls == 10]).all() and np.isnan(ref[:, cls == 11]).all()
        assert np.isinf(ref[:, cls == 12]).all()
        huge = ref[:, cls == 13]
        assert np.isfinite(huge).all() and (np.abs(huge) >= 2.0 ** 110).all()
        assert (ref[:, cls == 14] == 0).all()
        assert np.isfinite(ref[:, (cls <= 9) | (cls == 15)]).all()
        assert np.max(np.abs(ref[:, cls <= 9])) < 2.0 ** 126
    else:
        assert np.isnan(ref[:, (cls == 10) | (cls == 11)]).all()
        assert np.isfinite(ref[:, (cls <= 9) | (cls >= 12)]).all()
    worst = check_special(mode, got, ref, xval, wq, s, K)
    print(f"{mode} M={M} N={N} K={K} {xform}: worst {worst:.2f} ulp of the output scale", flush=True)
