"""GPU parity of the packed GDN recurrence (qmm_gdn_recurrence) against the oracle
(oracle/gdn.py), through the C ABI.

Cases: the reference's two tests (src/model.zig:1417-1446 hand-computed step,
zero-padded to Dk = 128; :1615-1706 pattern case with its bars and tighter
ones), the model's shapes (Hk 16, Hv 48, Dk = Dv = 128, bf16 q/k/v/beta, f32 g),
grouped heads with ragged Dv, a T split in two calls (the prefix/rest split of
gdnRecurFused, src/model.zig:343-390) equal bit for bit to one call, the state
updated in place, and the argument checks of fusedEligible (:322-329).

Bar: state within 1e-5 of the f64 oracle relative to its largest entry; y
within 1 bf16 ulp of the f64 value (plus 1e-5 of the row scale for the f32
accumulation).
"""
import numpy as np
import pytest

import oracle as O
import qmm as Q
from gdn import gdn_recurrence, reference_pattern_case

pytestmark = pytest.mark.gpu


def bf16(a):
    return O.f32_to_bf16_bits(np.asarray(a, np.float32))


def f32(bits):
    return O.bf16_bits_to_f32(bits)


def run(q, k, v, g, beta, st, *, in_dtype=Q.BFLOAT16, beta_dtype=Q.BFLOAT16, y_dtype=Q.BFLOAT16):
    """Inputs given as float arrays; bf16 inputs are rounded first (and the rounded
    values are what the oracle sees).  Returns y, state, and the inputs as used."""
    conv = (lambda a: bf16(a)) if in_dtype == Q.BFLOAT16 else (lambda a: np.asarray(a, np.float32))
    used = lambda a, dt: f32(a) if dt == Q.BFLOAT16 else a
    qa, ka, va = conv(q), conv(k), conv(v)
    ba = bf16(beta) if beta_dtype == Q.BFLOAT16 else np.asarray(beta, np.float32)
    A = Q.Array.from_numpy
    y, so = Q.gdn_recurrence(A(qa, in_dtype), A(ka, in_dtype), A(va, in_dtype), A(np.asarray(g, np.float32), Q.FLOAT32),
                             A(ba, beta_dtype), A(np.asarray(st, np.float32), Q.FLOAT32), y_dtype=y_dtype)
    yn = y.numpy()
    yn = f32(yn) if y_dtype == Q.BFLOAT16 else yn
    return yn, so.numpy(), (used(qa, in_dtype), used(ka, in_dtype), used(va, in_dtype), np.asarray(g, np.float32),
                            used(ba, beta_dtype), np.asarray(st, np.float32))


def check(y, S, inputs, y_bf16=True):
    yr, Sr = gdn_recurrence(*inputs)
    sscale = max(np.max(np.abs(Sr)), 1e-30)
    assert np.max(np.abs(S - Sr)) <= 1e-5 * sscale, np.max(np.abs(S - Sr)) / sscale
    rscale = np.max(np.abs(yr), axis=-1, keepdims=True)
    mag = np.abs(yr)
    ulp = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-38))) - 7), 0.0) if y_bf16 else 0.0
    bound = ulp + 1e-5 * rscale + 1e-30
    assert np.all(np.abs(y - yr) <= bound), np.max(np.abs(y - yr) / bound)


def model_inputs(rng, B, T, Hk, Hv, Dv, Dk=128, state_scale=0.1):
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    # the reference feeds RMS-normalised q / sqrt(Dk)^2 and k / sqrt(Dk) (src/model.zig:1110-1119)
    q = q / np.sqrt(np.mean(q * q, axis=-1, keepdims=True)) / Dk
    k = k / np.sqrt(np.mean(k * k, axis=-1, keepdims=True)) / np.sqrt(Dk)
    v = rng.standard_normal((B, T, Hv, Dv))
    g = np.exp(-rng.uniform(0.0, 0.7, (B, T, Hv))).astype(np.float32)  # exp(-softplus * A) in (0, 1)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv))))  # sigmoid
    st = (rng.standard_normal((B, Hv, Dv, Dk)) * state_scale).astype(np.float32)
    return q, k, v, g, beta, st


def test_reference_hand_computed_step_padded():
    """src/model.zig:1417-1446 (Dk = Dv = 2) embedded in Dk = 128, Dv = 8 with zeros."""
    q = np.zeros((1, 1, 1, 128)); q[..., :2] = [1, 2]
    k = np.zeros((1, 1, 1, 128)); k[..., :2] = [3, 4]
    v = np.zeros((1, 1, 1, 8)); v[..., :2] = [5, 6]
    g = np.full((1, 1, 1), 0.5); beta = np.ones((1, 1, 1))
    st = np.zeros((1, 1, 8, 128))
    for in_dt in (Q.BFLOAT16, Q.FLOAT32):
        y, S, _ = run(q, k, v, g, beta, st, in_dtype=in_dt, beta_dtype=in_dt)
        assert np.array_equal(y.reshape(8), [55, 66, 0, 0, 0, 0, 0, 0])
        Se = np.zeros((8, 128)); Se[:2, :2] = [[15, 20], [18, 24]]
        assert np.array_equal(S.reshape(8, 128), Se)


def test_reference_pattern_case():
    """src/model.zig:1615-1706: f32 inputs, bf16 y; its bars max |dy| < 0.05, max |dS| < 1e-3."""
    q, k, v, g, beta, st = reference_pattern_case()
    y, S, used = run(q, k, v, g, beta, st, in_dtype=Q.FLOAT32, beta_dtype=Q.FLOAT32)
    yr, Sr = gdn_recurrence(*used, acc="f32")
    assert np.max(np.abs(y - yr)) < 0.05 and np.max(np.abs(S - Sr)) < 1e-3
    check(y, S, used)


@pytest.mark.parametrize("T", [1, 3, 16, 37, 130])
def test_model_shapes(T):
    rng = np.random.default_rng(T)
    q, k, v, g, beta, st = model_inputs(rng, 1, T, 16, 48, 128)
    y, S, used = run(q, k, v, g, beta, st)
    check(y, S, used)


@pytest.mark.parametrize("B,T,Hk,Hv,Dv", [(2, 5, 2, 6, 24), (1, 19, 1, 2, 8), (3, 2, 4, 4, 136)])
@pytest.mark.parametrize("dtypes", ["bf16", "f32", "f32-beta-bf16-y-f32"])
def test_grouped_heads_ragged_rows(B, T, Hk, Hv, Dv, dtypes):
    rng = np.random.default_rng(B * 100 + T + Dv)
    q, k, v, g, beta, st = model_inputs(rng, B, T, Hk, Hv, Dv)
    kw = {"bf16": {}, "f32": dict(in_dtype=Q.FLOAT32, beta_dtype=Q.FLOAT32),
          "f32-beta-bf16-y-f32": dict(in_dtype=Q.FLOAT32, beta_dtype=Q.BFLOAT16, y_dtype=Q.FLOAT32)}[dtypes]
    y, S, used = run(q, k, v, g, beta, st, **kw)
    check(y, S, used, y_bf16=kw.get("y_dtype", Q.BFLOAT16) == Q.BFLOAT16)


def test_split_in_two_calls_is_bitwise_equal():
    """gdnRecurFused runs a confirmed prefix and the rest as two launches (src/model.zig:343-390)."""
    rng = np.random.default_rng(3)
    T, nc = 40, 17
    q, k, v, g, beta, st = model_inputs(rng, 1, T, 16, 48, 128)
    A = Q.Array.from_numpy
    qb, kb, vb, bb = bf16(q), bf16(k), bf16(v), bf16(beta)
    g32, s32 = g.astype(np.float32), st.astype(np.float32)
    y, S = Q.gdn_recurrence(A(qb, Q.BFLOAT16), A(kb, Q.BFLOAT16), A(vb, Q.BFLOAT16), A(g32, Q.FLOAT32),
                            A(bb, Q.BFLOAT16), A(s32, Q.FLOAT32))
    sl = lambda a, lo, hi: np.ascontiguousarray(a[:, lo:hi])
    parts, Sp = [], A(s32, Q.FLOAT32)
    for lo, hi in ((0, nc), (nc, T)):
        yp, Sp = Q.gdn_recurrence(A(sl(qb, lo, hi), Q.BFLOAT16), A(sl(kb, lo, hi), Q.BFLOAT16),
                                  A(sl(vb, lo, hi), Q.BFLOAT16), A(sl(g32, lo, hi), Q.FLOAT32),
                                  A(sl(bb, lo, hi), Q.BFLOAT16), Sp)
        parts.append(yp.numpy())
    assert np.array_equal(np.concatenate(parts, axis=1), y.numpy())
    assert np.array_equal(Sp.numpy(), S.numpy())


def test_state_in_place():
    rng = np.random.default_rng(4)
    q, k, v, g, beta, st = model_inputs(rng, 1, 2, 16, 48, 128)
    A = Q.Array.from_numpy
    args = (A(bf16(q), Q.BFLOAT16), A(bf16(k), Q.BFLOAT16), A(bf16(v), Q.BFLOAT16), A(g.astype(np.float32), Q.FLOAT32),
            A(bf16(beta), Q.BFLOAT16))
    s_a = A(st.astype(np.float32), Q.FLOAT32)
    y1, S1 = Q.gdn_recurrence(*args, A(st.astype(np.float32), Q.FLOAT32))
    y2, S2 = Q.gdn_recurrence(*args, s_a, state_out=s_a)
    assert S2.h.ctx == s_a.h.ctx  # the caller's array, updated in place
    assert np.array_equal(y1.numpy(), y2.numpy())
    assert np.array_equal(S1.numpy(), s_a.numpy())


def test_argument_checks():
    rng = np.random.default_rng(5)
    q, k, v, g, beta, st = model_inputs(rng, 1, 2, 2, 4, 16)
    A = Q.Array.from_numpy
    ok = dict(q=A(bf16(q), Q.BFLOAT16), k=A(bf16(k), Q.BFLOAT16), v=A(bf16(v), Q.BFLOAT16),
              g=A(g.astype(np.float32), Q.FLOAT32), beta=A(bf16(beta), Q.BFLOAT16), state=A(st, Q.FLOAT32))
    Q.gdn_recurrence(**ok)
    bad = [dict(g=A(bf16(g), Q.BFLOAT16)),  # fusedEligible: g must be f32
           dict(state=A(bf16(st), Q.BFLOAT16)),  # state f32
           dict(q=A(bf16(q[..., :64]), Q.BFLOAT16), k=A(bf16(k[..., :64]), Q.BFLOAT16),
                state=A(np.ascontiguousarray(st[..., :64]), Q.FLOAT32)),  # Dk != 128
           dict(v=A(bf16(v[..., :12]), Q.BFLOAT16), state=A(np.ascontiguousarray(st[:, :, :12]), Q.FLOAT32)),  # Dv % 8
           dict(q=A(q.astype(np.float32), Q.FLOAT32))]  # mixed input dtypes
    for b in bad:
        with pytest.raises(Q.QmmError):
            Q.gdn_recurrence(**{**ok, **b})


# The chunked form (T >= 96): chunks of 64 steps on the f32 MFMA, the last chunk
# padded with neutral steps; the same bar against the f64 oracle.
@pytest.mark.parametrize("T", [96, 128, 200, 1000, 2048])
def test_chunked_model_shapes(T):
    rng = np.random.default_rng(1000 + T)
    q, k, v, g, beta, st = model_inputs(rng, 1, T, 16, 48, 128)
    y, S, used = run(q, k, v, g, beta, st)
    check(y, S, used)


CHUNKED_KW = {"bf16": dict(),
              "bf16-y-f32": dict(y_dtype=Q.FLOAT32),
              "f32": dict(in_dtype=Q.FLOAT32, beta_dtype=Q.FLOAT32),
              "f32-beta-bf16-y-f32": dict(in_dtype=Q.FLOAT32, beta_dtype=Q.BFLOAT16, y_dtype=Q.FLOAT32)}


@pytest.mark.parametrize("dtypes", sorted(CHUNKED_KW))
def test_chunked_dtypes_and_batches(dtypes):
    rng = np.random.default_rng(77)
    q, k, v, g, beta, st = model_inputs(rng, 2, 150, 2, 6, 32)
    kw = CHUNKED_KW[dtypes]
    y, S, used = run(q, k, v, g, beta, st, **kw)
    check(y, S, used, y_bf16=kw.get("y_dtype", Q.BFLOAT16) == Q.BFLOAT16)


@pytest.mark.parametrize("dtypes", ["bf16", "f32"])
def test_chunked_grid_padding(dtypes):
    """6 scan workgroups (3 heads x 2 row groups): the grid is rounded up to 8 and the two
    extra workgroups exit; 130 steps leave a 2-step last chunk."""
    rng = np.random.default_rng(79)
    q, k, v, g, beta, st = model_inputs(rng, 1, 130, 1, 3, 32)
    kw = CHUNKED_KW[dtypes]
    y, S, used = run(q, k, v, g, beta, st, **kw)
    check(y, S, used, y_bf16=True)


def test_chunked_extreme_decays_and_gates():
    """Decays of exactly 1 and 0 (the state wiped mid-chunk) and tiny ones, gates of 0 and 1."""
    rng = np.random.default_rng(78)
    T = 300
    q, k, v, g, beta, st = model_inputs(rng, 1, T, 4, 8, 128)
    g[:, 10:20] = 1.0
    g[:, 70] = 0.0
    g[:, 100:110] = 1e-3
    g[:, 200] = 0.0
    beta[:, 30:40] = 0.0
    beta[:, 40:50] = 1.0
    y, S, used = run(q, k, v, g, beta, st)
    check(y, S, used)


def test_chunked_state_in_place():
    rng = np.random.default_rng(79)
    q, k, v, g, beta, st = model_inputs(rng, 1, 200, 16, 48, 128)
    A = Q.Array.from_numpy
    args = (A(bf16(q), Q.BFLOAT16), A(bf16(k), Q.BFLOAT16), A(bf16(v), Q.BFLOAT16), A(g.astype(np.float32), Q.FLOAT32),
            A(bf16(beta), Q.BFLOAT16))
    s_a = A(st.astype(np.float32), Q.FLOAT32)
    y1, S1 = Q.gdn_recurrence(*args, A(st.astype(np.float32), Q.FLOAT32))
    y2, S2 = Q.gdn_recurrence(*args, s_a, state_out=s_a)
    assert S2.h.ctx == s_a.h.ctx
    assert np.array_equal(y1.numpy(), y2.numpy())
    assert np.array_equal(S1.numpy(), s_a.numpy())


def test_long_T_rows_not_multiple_of_16_step_kernel():
    """Dv = 24 (not a multiple of the chunked form's 16 rows): the step-by-step kernel."""
    rng = np.random.default_rng(80)
    q, k, v, g, beta, st = model_inputs(rng, 1, 160, 2, 4, 24)
    y, S, used = run(q, k, v, g, beta, st)
    check(y, S, used)


@pytest.mark.parametrize("T", [95, 96, 200])
def test_nan_decay_propagates(T):
    """A NaN g at one step of one head: NaN in that head's y from the step on and in its
    state, in the step kernel (T < 96) and in the chunked form (T >= 96), where it also
    reaches the earlier steps of its 64-step chunk; every other head stays finite."""
    rng = np.random.default_rng(T)
    q, k, v, g, beta, st = model_inputs(rng, 1, T, 2, 6, 16)
    g[0, 70 if T > 96 else 40, 3] = np.nan
    t_nan = 70 if T > 96 else 40
    y, S, _ = run(q, k, v, g, beta, st)
    assert np.isnan(y[0, t_nan:, 3]).all() and np.isnan(S[0, 3]).all()
    others = [h for h in range(6) if h != 3]
    assert np.isfinite(y[..., others, :]).all() and np.isfinite(S[:, others]).all()
    first = t_nan if T < 96 else t_nan // 64 * 64  # steps before this one are finite
    assert np.isfinite(y[0, :first, 3]).all()
