"""Pins the CPU oracle (oracle/lizard_oracle.py) before it is trusted.

Every vectorised oracle function is checked against an independent closed
form (explicit loops written from the formula, as the reference's own ground
truth in tests/test_lizard.py:22-91 does), against invariants the math fixes
(gate 0 -> v, constant v, softmax limit == a library routine, sinks algebra),
and against finite differences.  ``test_checks_catch_planted_mistakes`` plants
plausible mistakes in copies of the oracle and asserts these checks fail them.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import lizard_oracle as lo

EXACT = 1e-10


def rel_err(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm()).item()


@pytest.fixture(autouse=True)
def seed():
    torch.manual_seed(0)


def gla_inputs(length, batch=2, heads=3, features=6, dim=5):
    fq = torch.randn(batch, heads, length, features).softmax(-1).double()
    fk = torch.randn(batch, heads, length, features).softmax(-1).double()
    v = torch.randn(batch, heads, length, dim).double()
    gamma = torch.sigmoid(2 * torch.randn(batch, length)).double()
    return fq, fk, v, gamma


def awa_inputs(length, batch=2, heads=3, dim=8, sinks=4):
    q, k, v = (torch.randn(batch, heads, length, dim).double() for _ in range(3))
    return q, k, v, torch.randn(sinks).double()


# -- window mask and gate products ------------------------------------------

@pytest.mark.parametrize("length, window", [(1, 1), (7, 3), (12, 12), (9, 100)])
def test_window_mask_is_the_predicate(length, window):
    mask = lo.window_mask(length, window)
    for i in range(length):
        for t in range(length):
            assert bool(mask[i, t]) == (t <= i and i - t < window)


def test_gate_products_brute_force():
    gamma = torch.rand(2, 9).double()
    d = lo.gate_products(gamma)
    for b in range(2):
        for i in range(9):
            for t in range(9):
                want = math.prod(gamma[b, t + 1:i + 1].tolist()) if t <= i else 0.0
                assert abs(d[b, i, t].item() - want) < 1e-15


# -- GLA --------------------------------------------------------------------

@pytest.mark.parametrize("length", [1, 5, 23])
def test_gla_matches_formula_loops(length):
    fq, fk, v, gamma = gla_inputs(length)
    assert rel_err(lo.gla(fq, fk, v, gamma), lo.gla_loop(fq, fk, v, gamma)) < EXACT


@pytest.mark.parametrize("length", [1, 64, 150])
def test_gla_matches_recurrent_form(length):
    fq, fk, v, gamma = gla_inputs(length)
    assert rel_err(lo.gla(fq, fk, v, gamma), lo.gla_recurrent(fq, fk, v, gamma)) < EXACT


def test_gla_gate_zero_keeps_only_the_current_token():
    fq, fk, v, gamma = gla_inputs(30)
    assert rel_err(lo.gla(fq, fk, v, torch.zeros_like(gamma)), v) < EXACT


def test_gla_constant_values_stay_constant():
    fq, fk, v, gamma = gla_inputs(30)
    c = torch.full_like(v, 0.37)
    assert rel_err(lo.gla(fq, fk, c, gamma), c) < EXACT


def test_gla_single_token_is_v():
    fq, fk, v, gamma = gla_inputs(1)
    assert rel_err(lo.gla(fq, fk, v, gamma), v) < EXACT


def test_gla_gate_one_is_normalised_causal_linear_attention():
    fq, fk, v, gamma = gla_inputs(17)
    w = (fq @ fk.transpose(-1, -2)).tril()
    expected = (w @ v) / w.sum(-1, keepdim=True)
    assert rel_err(lo.gla(fq, fk, v, torch.ones_like(gamma)), expected) < EXACT


def test_gla_kernel_api_per_token_and_per_head_agree():
    fq, fk, v, gamma = gla_inputs(20)
    lg = torch.log(gamma)
    per_token = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    per_head = lo.gla_kernel_api(fq, fk, v, lg[:, None].expand(-1, 3, -1),
                                 dtype=torch.float64)
    assert rel_err(per_token, per_head) < EXACT
    assert rel_err(per_token, lo.gla_loop(fq, fk, v, gamma)) < EXACT


def test_gla_kernel_api_per_head_gates_are_per_head():
    fq, fk, v, _ = gla_inputs(12, batch=1, heads=2)
    lg = F.logsigmoid(torch.randn(1, 2, 12)).double()
    y = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    for h in range(2):
        ref = lo.gla_loop(fq[:, h:h + 1], fk[:, h:h + 1], v[:, h:h + 1], lg[:, h].exp())
        assert rel_err(y[:, h:h + 1], ref) < EXACT


# -- window softmax with sinks ---------------------------------------------

@pytest.mark.parametrize("length", [1, 15, 16, 17, 70])
def test_awa_matches_formula_loops(length):
    q, k, v, meta = awa_inputs(length)
    assert rel_err(lo.awa(q, k, v, meta, 16), lo.awa_loop(q, k, v, meta, 16)) < EXACT


def test_awa_without_sinks_and_window_is_causal_softmax():
    q, k, v, _ = awa_inputs(40)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    no_sinks = torch.full((4,), -1e4).double()
    assert rel_err(lo.awa(q, k, v, no_sinks, 10 ** 6), expected) < EXACT
    assert rel_err(lo.awa(q, k, v, torch.empty(0).double(), 10 ** 6), expected) < EXACT


def test_awa_many_sinks_equal_one_sink_with_logsumexp():
    q, k, v, meta = awa_inputs(40)
    one = torch.logsumexp(meta, 0, keepdim=True)
    assert rel_err(lo.awa(q, k, v, meta, 16), lo.awa(q, k, v, one, 16)) < EXACT


def test_awa_window_one_is_a_scaled_copy_of_v():
    q, k, v, meta = awa_inputs(10)
    s = (q * k).sum(-1, keepdim=True) / math.sqrt(q.shape[-1])
    expected = v * torch.exp(s) / (torch.exp(s) + meta.exp().sum())
    assert rel_err(lo.awa(q, k, v, meta, 1), expected) < EXACT


def test_empty_meta_equals_very_negative_sink():
    q, k, v, _ = awa_inputs(40)
    a = lo.swa_kernel_api(q, k, v, torch.empty(0), 16, dtype=torch.float64)
    b = lo.swa_kernel_api(q, k, v, torch.full((1,), -1e4), 16, dtype=torch.float64)
    assert rel_err(a, b) < EXACT


# -- gradients, causality ---------------------------------------------------

@pytest.mark.parametrize("fn", ["hedgehog", "gla", "awa"])
def test_gradients_match_finite_differences(fn):
    if fn == "hedgehog":
        args, call = (torch.randn(1, 2, 4, 5), torch.randn(3, 5)), lo.hedgehog
    elif fn == "gla":
        args, call = gla_inputs(6, batch=1, heads=2, features=3, dim=2), lo.gla
    else:
        args = awa_inputs(6, batch=1, heads=2, dim=3)
        call = lambda *a: lo.awa(*a, 3)  # noqa: E731
    args = [a.double().requires_grad_() for a in args]
    assert torch.autograd.gradcheck(call, args)


def test_gla_kernel_api_gate_gradient_matches_finite_differences():
    fq, fk, v, _ = gla_inputs(9, batch=1, heads=2, features=3, dim=2)
    for shape in ((1, 9), (1, 2, 9)):
        lg = F.logsigmoid(torch.randn(*shape)).double().requires_grad_()
        call = lambda g: lo.gla_kernel_api(fq, fk, v, g, dtype=torch.float64)  # noqa: E731
        assert torch.autograd.gradcheck(call, (lg,))


@pytest.mark.parametrize("branch", ["gla", "awa"])
def test_branch_has_zero_gradient_from_future_tokens(branch):
    inputs = gla_inputs(20) if branch == "gla" else awa_inputs(20)
    q, k, v, extra = [t.requires_grad_() for t in inputs]
    out = lo.gla(q, k, v, extra) if branch == "gla" else lo.awa(q, k, v, extra, 16)
    out[:, :, 9].sum().backward()
    for grad in (q.grad, k.grad, v.grad):
        assert (grad[:, :, 10:] == 0).all()


def test_awa_has_gradient_only_inside_the_window():
    q, k, v, meta = [t.requires_grad_() for t in awa_inputs(40)]
    lo.awa(q, k, v, meta, 16)[:, :, 39].sum().backward()
    assert (k.grad[:, :, :24] == 0).all()
    assert (k.grad[:, :, 24:].abs().sum(-1) > 0).all()


# -- hedgehog, rope ----------------------------------------------------------

def test_hedgehog_matches_formula():
    x, w = torch.randn(2, 3, 20, 16).double(), torch.randn(8, 16).double()
    assert rel_err(lo.hedgehog(x, w), lo.hedgehog_loop(x, w)) < EXACT
    halves = lo.hedgehog(x, w).view(2, 3, 20, 2, 8).sum(-1)
    assert torch.allclose(halves, torch.ones(1).double())


def test_rope_matches_loop_and_is_relative():
    cos, sin = lo.rope_cos_sin(20, 8, theta=500000.0)
    x = torch.randn(2, 3, 20, 8).double()
    assert rel_err(lo.rope(x, cos, sin), lo.rope_loop(x, cos, sin)) < EXACT
    q, k = torch.randn(8).double(), torch.randn(8).double()
    cos2, sin2 = lo.rope_cos_sin(40, 8, theta=500000.0)
    dots = [(lo.rope(q, cos2[p + 5], sin2[p + 5]) * lo.rope(k, cos2[p], sin2[p])).sum()
            for p in (0, 7, 30)]
    assert max(abs(d - dots[0]) for d in dots) < 1e-12


# -- chunked restatement == dense -------------------------------------------

@pytest.mark.parametrize("length, chunk", [(1, 16), (77, 16), (150, 64), (130, 64)])
def test_chunked_equals_dense(length, chunk):
    fq, fk, v, gamma = gla_inputs(length, features=24, dim=20)
    lg = torch.log(gamma)
    dense = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    assert rel_err(lo.gla_chunked(fq, fk, v, lg, chunk), dense) < EXACT


def test_chunked_equals_dense_per_head_and_strong_decay():
    fq, fk, v, _ = gla_inputs(200, features=24, dim=20)
    lg = F.logsigmoid(2 * torch.randn(2, 3, 200) - 6.0).double()
    assert lg.sum(-1).max() < -1000
    dense = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    assert rel_err(lo.gla_chunked(fq, fk, v, lg, 64), dense) < EXACT
    assert rel_err(lo.gla_chunked(fq, fk, v, lg, 16), dense) < EXACT


def test_chunked_bf16_emulation_stays_close():
    fq, fk, v, gamma = gla_inputs(300, features=64, dim=64)
    lg = torch.log(gamma)
    dense = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    emu = lo.gla_chunked(fq, fk, v, lg, 64, round_bf16=True)
    assert (emu - dense).abs().max() / dense.abs().max() < 1e-2


# -- the checks have teeth: planted mistakes fail them ----------------------

_GOOD_GATE_PRODUCTS = lo.gate_products


def _mutant_gate_products_off_by_one(gamma):
    # includes gamma_t itself in the product (a wrong index)
    return _GOOD_GATE_PRODUCTS(gamma) * gamma.unsqueeze(-2)


def _mutant_window(length, window, device=None):
    rows = torch.arange(length).unsqueeze(1)
    cols = torch.arange(length).unsqueeze(0)
    return (cols <= rows) & ((rows - cols) <= window)   # one key too many


def test_checks_catch_planted_mistakes(monkeypatch):
    fq, fk, v, gamma = gla_inputs(12)
    good = lo.gla(fq, fk, v, gamma)
    with monkeypatch.context() as m:
        m.setattr(lo, "gate_products", _mutant_gate_products_off_by_one)
        assert rel_err(lo.gla(fq, fk, v, gamma), lo.gla_loop(fq, fk, v, gamma)) > 1e-3
    # transposed operand: fk^T fq instead of fq fk^T
    wrong = (fk @ fq.transpose(-1, -2)) * lo.gate_products(gamma).unsqueeze(1)
    wrong = (wrong @ v) / wrong.sum(-1, keepdim=True)
    assert rel_err(wrong, good) > 1e-3
    q, k, vv, meta = awa_inputs(30)
    with monkeypatch.context() as m:
        m.setattr(lo, "window_mask", _mutant_window)
        assert rel_err(lo.awa(q, k, vv, meta, 8), lo.awa_loop(q, k, vv, meta, 8)) > 1e-3
    # a dropped sink term
    no_sink = lo.awa(q, k, vv, torch.empty(0).double(), 8)
    assert rel_err(no_sink, lo.awa_loop(q, k, vv, meta, 8)) > 1e-3
    # wrong sign of the chunk decay in the chunked restatement
    lg = torch.log(gamma)
    dense = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    assert rel_err(lo.gla_chunked(fq, fk, v, -lg.abs() * 0.5, 4), dense) > 1e-3


# -- recurrent state (decode form) ----------------------------------------------

@pytest.mark.parametrize("per_head", [False, True])
def test_recurrent_state_matches_recurrent_form_and_chunked_state(per_head):
    fq, fk, v, gamma = gla_inputs(70, features=12, dim=10)
    if per_head:
        gamma = torch.sigmoid(2 * torch.randn(2, 3, 70)).double()
    out, S, z = lo.gla_recurrent_state(fq, fk, v, gamma)
    lg = torch.log(gamma)
    dense = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float64)
    assert rel_err(out, dense) < EXACT
    if not per_head:
        assert rel_err(out, lo.gla_recurrent(fq, fk, v, gamma)) < EXACT
    for chunk in (16, 64):
        c_out, c_S, c_z = lo.gla_chunked(fq, fk, v, lg, chunk, return_state=True)
        assert rel_err(c_S, S) < EXACT and rel_err(c_z, z) < EXACT
        assert rel_err(c_out, dense) < EXACT


def test_recurrent_state_continues_a_prefix():
    """Running the recurrence on a prefix, then on the rest from that state,
    gives the whole sequence's outputs: what decoding after a prefill does."""
    fq, fk, v, gamma = gla_inputs(40, features=8, dim=6)
    full, S_full, z_full = lo.gla_recurrent_state(fq, fk, v, gamma)
    _, S, z = lo.gla_recurrent_state(fq[:, :, :25], fk[:, :, :25], v[:, :, :25], gamma[:, :25])
    for i in range(25, 40):
        g = gamma[:, i].view(-1, 1, 1)
        S = g[..., None] * S + fk[:, :, i, :, None] * v[:, :, i, None, :]
        z = g * z + fk[:, :, i]
        y = (fq[:, :, i, :, None] * S).sum(-2) / (fq[:, :, i] * z).sum(-1, keepdim=True)
        assert rel_err(y, full[:, :, i]) < EXACT
    assert rel_err(S, S_full) < EXACT and rel_err(z, z_full) < EXACT
