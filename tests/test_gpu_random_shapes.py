"""Seeded random shapes through the operator API, against the CPU oracle.

The fixed-shape tests pin each code path on purpose; this sweep draws the
arguments the reference operators accept (src/kernels/gla.py:259-263,
src/kernels/swa.py:182-183) in combinations nobody picked by hand: ragged
lengths from 1 up, feature and value widths off the tile sizes, per-token and
per-head gates with strong and weak decay, fp32 or bf16 inputs, windows from 1
past the sequence, and 0 to 70 sink logits.  Every case is checked like the
fixed ones: output and every gradient within the bar of the fp32 oracle, and
gradients in the inputs' dtype.
"""
import random

import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import GRAD_TOL, OUT_TOL, compare, max_rel

pytestmark = pytest.mark.gpu


def _gla_cases(n, seed=20261202):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        cases.append(dict(
            batch=rng.choice([1, 2, 3]), heads=rng.choice([1, 2, 3, 5]),
            length=rng.choice([1, 2, 63, 64, 65]) if i % 5 == 0 else rng.randint(3, 600),
            features=rng.choice([8, 24, 32, 48, 64, 100, 128, 160, 256, 264]),
            dim=rng.choice([8, 20, 32, 64, 72, 128, 136]),
            per_head=rng.random() < 0.5, shift=rng.choice([-2.0, 0.0, 3.0]),
            fp32=rng.random() < 0.3, seed=rng.randint(0, 10 ** 6)))
    return cases


def _swa_cases(n, seed=1202):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        length = rng.choice([1, 2, 31]) if i % 5 == 0 else rng.randint(3, 600)
        cases.append(dict(
            batch=rng.choice([1, 2, 3]), heads=rng.choice([1, 2, 3, 5]), length=length,
            dim=rng.choice([8, 16, 20, 32, 40, 64, 80, 96, 128, 192, 256]),
            window=rng.choice([1, 2, 7, 33, 64, 65, 128, 257, length + 5]),
            sinks=rng.choice([0, 1, 4, 7, 65, 70]),
            fp32=rng.random() < 0.3, seed=rng.randint(0, 10 ** 6)))
    return cases


def _label(case):
    return ",".join(f"{k}={v}" for k, v in case.items() if k != "seed")


GLA_CASES = _gla_cases(40)
SWA_CASES = _swa_cases(40)


@pytest.mark.parametrize("case", GLA_CASES, ids=[_label(c) for c in GLA_CASES])
def test_gla_random_shape_matches_oracle(case):
    g = torch.Generator().manual_seed(case["seed"])
    b, h, length = case["batch"], case["heads"], case["length"]
    dtype = torch.float32 if case["fp32"] else torch.bfloat16
    # features as the reference's tests draw them (softmax rows), rounded to
    # bf16 first so that both sides see the same values whatever the dtype
    fq = torch.randn(b, h, length, case["features"], generator=g).softmax(-1).bfloat16().to(dtype)
    fk = torch.randn(b, h, length, case["features"], generator=g).softmax(-1).bfloat16().to(dtype)
    v = torch.randn(b, h, length, case["dim"], generator=g).bfloat16().to(dtype)
    z = 2 * torch.randn(*((b, h, length) if case["per_head"] else (b, length)), generator=g) \
        + case["shift"]
    grad = torch.randn(b, h, length, case["dim"], generator=g)
    if length == 1:
        _check_gla_single_token(fq, fk, v, z, grad, "gla " + _label(case))
        return
    compare(lambda a, c, d, e: kernels.gla(a, c, d, F.logsigmoid(e)),
            lambda a, c, d, e: lo.gla_kernel_api(a, c, d, F.logsigmoid(e), dtype=torch.float32),
            [fq, fk, v, z], grad, label="gla " + _label(case))


def _check_gla_single_token(fq, fk, v, z, grad, label):
    """L = 1: y = v exactly, dv = dy, and dfq, dfk, d log_gamma vanish.

    dfq is the difference of two equal terms, fk (dy.v) / w and fk (dy.y) / w
    with w = fq.fk (dfk the same with fq), so what comes out is their rounding
    noise, and its size follows the terms: with softmax features over F
    columns, w ~ 1/F and the terms grow with F.  The relative check of the
    other cases divides that noise by a fixed floor; here it is measured
    against the terms themselves (the oracle's fp32 noise is of the same kind).
    d log_gamma = fq.dfq - fk.dfk is measured against dy.v, the size of each
    of its two terms (fq.fk / w = 1).
    """
    leaves = [t.detach().clone().cuda().requires_grad_() for t in (fq, fk, v, z)]
    y = kernels.gla(leaves[0], leaves[1], leaves[2], F.logsigmoid(leaves[3]))
    dy = grad.to(y.dtype)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    q64, k64, v64, dy64 = (t.double() for t in (fq, fk, v, dy))
    w = (q64 * k64).sum(-1, keepdim=True)
    dyv = (dy64 * v64).sum(-1, keepdim=True).abs()
    term_q = (k64.abs() * dyv / w).amax().item()   # size of the terms in dfq
    term_k = (q64.abs() * dyv / w).amax().item()
    report = {"out": max_rel(y, v64), "dv": max_rel(leaves[2].grad, dy64),
              "dfq/term": leaves[0].grad.double().abs().max().item() / term_q,
              "dfk/term": leaves[1].grad.double().abs().max().item() / term_k,
              "dz/term": leaves[3].grad.double().abs().max().item() / dyv.amax().item()}
    print(f"[parity] {label}: " + " ".join(f"{k}={x:.2e}" for k, x in report.items()), flush=True)
    assert y.dtype == torch.bfloat16 and leaves[0].grad.dtype == fq.dtype, label
    assert report["out"] <= OUT_TOL and report["dv"] <= GRAD_TOL, (label, report)
    assert report["dfq/term"] <= 1e-4 and report["dfk/term"] <= 1e-4, (label, report)
    assert report["dz/term"] <= 1e-4, (label, report)


@pytest.mark.parametrize("case", SWA_CASES, ids=[_label(c) for c in SWA_CASES])
def test_swa_random_shape_matches_oracle(case):
    g = torch.Generator().manual_seed(case["seed"])
    b, h, length, d = case["batch"], case["heads"], case["length"], case["dim"]
    dtype = torch.float32 if case["fp32"] else torch.bfloat16
    q, k, v = (torch.randn(b, h, length, d, generator=g).bfloat16().to(dtype) for _ in range(3))
    meta = torch.randn(case["sinks"], generator=g)
    grad = torch.randn(b, h, length, d, generator=g)
    w = case["window"]
    compare(lambda a, c, e, m: kernels.swa(a, c, e, m, w),
            lambda a, c, e, m: lo.swa_kernel_api(a, c, e, m, w, dtype=torch.float32),
            [q, k, v, meta], grad, label="swa " + _label(case))
