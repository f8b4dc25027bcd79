"""GPU parity of the HIP SWA path against the CPU oracle.

Mirrors the reference's kernel tests (tests/test_kernels.py:110-134):
(L, W) in {(1, 8), (77, 32), (150, 128)}, small and default blocks, no sinks,
plus BASELINE config 3 (B=1, H=32, L=2048, d=64, W=64, 4 sink logits, RoPE'd
q and k) against the dense oracle.
"""
import pytest
import torch

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import (GRAD_TOL, OUT_TOL, baseline_swa_inputs, compare, max_rel,
                           norm_rel, swa_inputs)

pytestmark = pytest.mark.gpu
SMALL = ((16, 16), (16, 16))


# W = 66 is the widest window whose key tiles the dq kernel keeps resident in
# LDS (at d <= 64); W = 67 streams them twice
@pytest.mark.parametrize("length, window, blocks", [(1, 8, SMALL), (77, 32, SMALL),
                                                    (150, 128, None), (300, 64, None),
                                                    (130, 1, None), (97, 200, None),
                                                    (333, 66, None), (333, 67, None)])
def test_swa_matches_oracle(length, window, blocks):
    inputs = swa_inputs(length)
    blocks = blocks or (kernels.FWD_BLOCKS, kernels.BWD_BLOCKS)

    def kernel(q, k, v, meta):
        return kernels.swa(q, k, v, meta, window, *blocks)

    def reference(q, k, v, meta):
        return lo.swa_kernel_api(q, k, v, meta, window, dtype=torch.float32)

    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(kernel, reference, inputs, grad, label=f"L={length} W={window}")


@pytest.mark.parametrize("dim", [32, 64, 128, 256])
def test_swa_head_dims(dim):
    inputs = swa_inputs(100, batch=1, heads=2, dim=dim)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(lambda q, k, v, m: kernels.swa(q, k, v, m, 48),
            lambda q, k, v, m: lo.swa_kernel_api(q, k, v, m, 48, dtype=torch.float32),
            inputs, grad, label=f"d={dim}")


def test_swa_without_sinks_matches_oracle():
    q, k, v, _ = swa_inputs(40)
    meta = torch.empty(0)
    y = kernels.swa(q.cuda(), k.cuda(), v.cuda(), meta.cuda(), 16, *SMALL)
    expected = lo.swa_kernel_api(q, k, v, torch.full((1,), -1e4), 16, dtype=torch.float32)
    assert norm_rel(y, expected) < 1e-2
    assert max_rel(y, expected) <= OUT_TOL


def test_swa_without_sinks_gradients():
    inputs = swa_inputs(90, sinks=0)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(lambda q, k, v, m: kernels.swa(q, k, v, m, 32),
            lambda q, k, v, m: lo.swa_kernel_api(q, k, v, m, 32, dtype=torch.float32),
            inputs, grad, label="no sinks")


def test_swa_is_deterministic():
    q, k, v, meta = (t.cuda().requires_grad_() for t in swa_inputs(200))
    outs = []
    for _ in range(2):
        y = kernels.swa(q, k, v, meta, 64)
        y.backward(torch.ones_like(y))
        outs.append([y.detach().clone()] + [t.grad.clone() for t in (q, k, v, meta)])
        for t in (q, k, v, meta):
            t.grad = None
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_swa_baseline_config3_dense():
    q, k, v, meta, dy = baseline_swa_inputs(1, 32, 2048, 64)
    ours = [t.cuda().requires_grad_() for t in (q, k, v, meta)]
    y = kernels.swa(*ours, 64)
    y.backward(dy.cuda())
    theirs = [t.clone().requires_grad_() for t in (q, k, v, meta)]
    ref = lo.swa_kernel_api(*theirs, 64, dtype=torch.float32)
    ref.backward(dy.float())
    errs = [max_rel(y, ref)] + [max_rel(a.grad, b.grad) for a, b in zip(ours, theirs)]
    print("SWA cfg3: out %.2e grads %s" % (errs[0], " ".join(f"{e:.2e}" for e in errs[1:])),
          flush=True)
    assert errs[0] <= OUT_TOL, errs
    assert max(errs[1:]) <= GRAD_TOL, errs


@pytest.mark.parametrize("dim", [20, 64])
def test_swa_fp32_inputs_give_fp32_grads_matching_oracle(dim):
    """fp32 q, k, v (what the reference's layer passes, src/lizard_attention.py:
    80-96): the output is bf16 and dq, dk, dv, dmeta come back fp32 (the
    kernels' fp32 gradient stores), within the bar of the fp32 oracle;
    d = 20 takes the element-wise path, d = 64 the 16-byte one."""
    inputs = swa_inputs(120, dim=dim)
    inputs = [t.float() for t in inputs[:3]] + [inputs[3]]
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    report = compare(lambda q, k, v, m: kernels.swa(q, k, v, m, 48),
                     lambda q, k, v, m: lo.swa_kernel_api(q, k, v, m, 48, dtype=torch.float32),
                     inputs, grad, label=f"fp32 inputs d={dim}")
    assert {"grad0", "grad1", "grad2", "grad3"} <= set(report)


@pytest.mark.parametrize("sinks, dim", [(100, 64), (300, 20)])
def test_swa_many_sinks_match_oracle(sinks, dim):
    """Any number of sink logits (the reference's BLOCK_S follows n_meta,
    src/kernels/swa.py:151-152): dmeta partials in passes of 64 sinks, their
    sum in passes of up to 256."""
    inputs = swa_inputs(150, dim=dim, sinks=sinks)
    inputs[3] = inputs[3] - 3.0   # keep the window's share of each row visible
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(lambda q, k, v, m: kernels.swa(q, k, v, m, 48),
            lambda q, k, v, m: lo.swa_kernel_api(q, k, v, m, 48, dtype=torch.float32),
            inputs, grad, label=f"{sinks} sinks d={dim}")
