"""qmm_gdn_recurrence_noalloc against qmm_gdn_recurrence, through the C ABI.

The allocation-free entry point runs the same kernels with the chunked form's
workspace in the library's static per-GPU array, so its results must equal the
allocating entry point's bit for bit, including when the workspace exceeds the
array and the call runs as several launches (batch groups, or runs of whole
64-step chunks).  Calls follow each other on a dirty array, the second smaller
than the first; every output starts as NaN, so an element never written fails.
"""
import pytest
import torch

import qmm as Q

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def inputs(B, T, Hk, Hv, Dv, seed, dtype=torch.bfloat16):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    rn = lambda *s: torch.randn(s, generator=gen, device=DEV, dtype=torch.float32)
    q, k = rn(B, T, Hk, 128), rn(B, T, Hk, 128)
    q = (q / q.pow(2).mean(-1, keepdim=True).sqrt() / 128).to(dtype)
    k = (k / k.pow(2).mean(-1, keepdim=True).sqrt() / 128 ** 0.5).to(dtype)
    v = rn(B, T, Hv, Dv).to(dtype)
    g = torch.exp(-0.7 * torch.rand((B, T, Hv), generator=gen, device=DEV))
    beta = torch.sigmoid(rn(B, T, Hv)).to(dtype)
    state = rn(B, Hv, Dv, 128) * 0.1
    return q, k, v, g, beta, state


def nan_like(shape, dtype):
    t = torch.empty(shape, dtype=dtype, device=DEV)
    t.view(torch.int16 if dtype == torch.bfloat16 else torch.int32).fill_(-1)  # all-ones bits: NaN
    return t


def run_both(B, T, Hk, Hv, Dv, seed, *, in_place=False, dtype=torch.bfloat16, y_dtype=Q.BFLOAT16):
    print(f"[noalloc] B={B} T={T} Hk={Hk} Hv={Hv} Dv={Dv} in_place={in_place} {dtype}", flush=True)
    q, k, v, g, beta, state = inputs(B, T, Hk, Hv, Dv, seed, dtype)
    A = Q.Array.from_torch
    tq, tk, tv, tg, tb = A(q), A(k), A(v), A(g), A(beta)
    ydt = torch.bfloat16 if y_dtype == Q.BFLOAT16 else torch.float32
    # the allocating entry point
    y_ref, s_ref = nan_like((B, T, Hv, Dv), ydt), state.clone()
    Q.gdn_recurrence(tq, tk, tv, tg, tb, A(s_ref), y=A(y_ref), state_out=A(s_ref), y_dtype=y_dtype)
    # the allocation-free one, into preallocated NaN-filled results
    y = nan_like((B, T, Hv, Dv), ydt)
    if in_place:
        s_in = state.clone()
        s_out = s_in
        sa = A(s_in)
        Q.gdn_recurrence_noalloc(tq, tk, tv, tg, tb, sa, y=A(y), state_out=sa, y_dtype=y_dtype)
    else:
        s_in = state.clone()
        s_out = nan_like((B, Hv, Dv, 128), torch.float32)
        Q.gdn_recurrence_noalloc(tq, tk, tv, tg, tb, A(s_in), y=A(y), state_out=A(s_out), y_dtype=y_dtype)
        assert torch.equal(s_in, state), "the input state changed"
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(s_out).all(), "an output element was not written"
    assert torch.equal(y.view(torch.int16 if ydt == torch.bfloat16 else torch.int32),
                       y_ref.view(torch.int16 if ydt == torch.bfloat16 else torch.int32)), "y differs"
    assert torch.equal(s_out.view(torch.int32), s_ref.view(torch.int32)), "state differs"


def test_batch_groups_then_smaller():
    # 2 x 48 heads x 32 chunks exceed the 2016 chunks the array holds: two launches of one batch
    run_both(2, 2048, 16, 48, 128, 1)
    run_both(1, 300, 16, 48, 128, 2)  # one launch, on the array the first call left dirty


def test_chunk_runs_then_smaller():
    # 48 heads x 65 chunks in one batch: runs of 42 chunks (2688 steps) carry the state
    run_both(1, 4133, 16, 48, 128, 3, in_place=True)
    run_both(1, 96, 16, 48, 128, 4)


def test_f32_inputs_and_outputs_and_step_kernel():
    run_both(3, 1500, 4, 8, 64, 5, dtype=torch.float32, y_dtype=Q.FLOAT32)
    run_both(2, 7, 16, 48, 128, 6)  # T < 96: the step kernel, no workspace


def test_rejections_allocate_nothing():
    q, k, v, g, beta, state = inputs(1, 100, 16, 48, 128, 7)
    A = Q.Array.from_torch
    args = [A(t) for t in (q, k, v, g, beta, state)]
    with pytest.raises(Q.QmmError, match="allocates nothing"):
        Q.gdn_recurrence_noalloc(*args, y=Q.Array(), state_out=A(state.clone()))
    with pytest.raises(Q.QmmError, match="allocates nothing"):
        Q.gdn_recurrence_noalloc(*args, y=A(nan_like((1, 99, 48, 128), torch.bfloat16)), state_out=A(state.clone()))
    with pytest.raises(Q.QmmError, match="allocates nothing"):
        Q.gdn_recurrence_noalloc(*args, y=A(nan_like((1, 100, 48, 128), torch.float32)), state_out=A(state.clone()))
    # one 64-step chunk over 2048 value heads needs more than the static array holds
    q, k, v, g, beta, state = inputs(1, 96, 1, 2048, 16, 8)
    y = nan_like((1, 96, 2048, 16), torch.bfloat16)
    with pytest.raises(Q.QmmError, match="static workspace"):
        Q.gdn_recurrence_noalloc(A(q), A(k), A(v), A(g), A(beta), A(state), y=A(y), state_out=A(state))
    torch.cuda.synchronize()
    assert torch.isnan(y.float()).all(), "a rejected call wrote its output"
