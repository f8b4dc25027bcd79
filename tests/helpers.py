"""Shared helpers of the parity tests: metrics, seeded input generators and a
``compare`` that runs the HIP path and the CPU oracle on cloned leaves with
the same upstream gradient (the shape of the reference's
tests/test_kernels.py:18-42)."""
import math

import torch
import torch.nn.functional as F

# max-abs error relative to the max-abs of the fp32 oracle
OUT_TOL, GRAD_TOL = 1e-2, 2e-2
# the reference's own bar (tests/test_kernels.py:15,18-25)
REF_FORWARD, REF_BACKWARD, REF_ATOL = 1e-2, 3e-2, 1e-3


# Floor of the scale in max_rel.  A gradient that is mathematically zero (at
# L=1, y = v exactly, so d/dfq, d/dfk and d/dlog_gamma vanish) comes out of
# both sides as ~1e-5 of rounding noise, and a ratio of two noises says
# nothing; every gradient of the test inputs that is not zero is >= 0.18 in
# max-abs, so the floor never loosens a real comparison.
SCALE_FLOOR = 1e-3


def max_rel(a, b, floor=SCALE_FLOOR):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    scale = max(b.abs().max().item() if b.numel() else 0.0, floor)
    return (a - b).abs().max().item() / scale if a.numel() else 0.0


def norm_rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


def ref_close(a, b, tol=REF_BACKWARD):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return (a - b).norm() <= tol * b.norm() + REF_ATOL * b.numel() ** 0.5


def leaves(tensors, device):
    return [t.detach().clone().to(device).requires_grad_() for t in tensors]


def compare(kernel, reference, inputs, grad, out_tol=OUT_TOL, grad_tol=GRAD_TOL, label=""):
    """kernel runs on the GPU, reference (the oracle) on the CPU, both from the
    same CPU-generated inputs; returns the error report."""
    ours = leaves(inputs, "cuda")
    theirs = leaves(inputs, "cpu")
    y = kernel(*ours)
    # The op's output is bf16, so autograd hands it the upstream gradient
    # rounded to bf16; the oracle gets that same rounded gradient, so that the
    # comparison measures the kernels and not the rounding of their input.
    # (The reference's harness gives its oracle the unrounded one,
    # tests/test_kernels.py:35-37; that rounding alone moves the sink gradient
    # by 2.5e-2 at d=32 in an fp64 computation.)
    dy = grad.to(y.dtype)
    y.backward(dy.to("cuda"))
    expected = reference(*theirs)
    expected.backward(dy.to(expected.dtype))
    torch.cuda.synchronize()
    report = {"out": max_rel(y, expected), "out_norm": norm_rel(y, expected)}
    for i, (a, b) in enumerate(zip(ours, theirs)):
        if b.grad is not None:
            report[f"grad{i}"] = max_rel(a.grad, b.grad)
    print(f"[parity] {label}: " + " ".join(f"{k}={v:.2e}" for k, v in report.items()),
          flush=True)
    assert y.dtype == torch.bfloat16, label
    assert report["out"] <= out_tol, (label, report)
    assert report["out_norm"] < REF_FORWARD, (label, report)
    for i, (a, b) in enumerate(zip(ours, theirs)):
        if b.grad is None:
            continue
        assert a.grad.dtype == b.dtype, (label, i, a.grad.dtype, b.dtype)
        assert report[f"grad{i}"] <= grad_tol, (label, i, report)
        assert ref_close(a.grad, b.grad), (label, i, report)
    return report


def gla_inputs(length, gates=(), shift=0.0, batch=2, heads=3, features=24, dim=20, seed=0):
    """The reference's GLA test inputs (tests/test_kernels.py:45-52): softmax
    features, N(0,1) values, gate logits z = 2 N(0,1) + shift."""
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    fq = torch.randn(batch, heads, length, features, generator=g).softmax(-1).to(bf)
    fk = torch.randn(batch, heads, length, features, generator=g).softmax(-1).to(bf)
    v = torch.randn(batch, heads, length, dim, generator=g).to(bf)
    z = 2 * torch.randn(batch, *gates, length, generator=g) + shift
    return [fq, fk, v, z]


def swa_inputs(length, batch=2, heads=3, dim=20, sinks=4, seed=0):
    """The reference's SWA test inputs (tests/test_kernels.py:73-76)."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(batch, heads, length, dim, generator=g).to(torch.bfloat16)
               for _ in range(3))
    return [q, k, v, torch.randn(sinks, generator=g)]


def baseline_gla_inputs(batch, heads, length, dim, per_head=False, gate_mean=3.0,
                        gate_std=1.0, seed=0):
    """BASELINE configs 1, 2, 4: fq, fk = softplus(N(0,1)), v = N(0,1) in bf16,
    log_gamma = logsigmoid(N(mean, std)) fp32 ([B, L] or [B, H, L]), dO = N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    shape = (batch, heads, length, dim)
    fq = F.softplus(torch.randn(shape, generator=g)).to(torch.bfloat16)
    fk = F.softplus(torch.randn(shape, generator=g)).to(torch.bfloat16)
    v = torch.randn(shape, generator=g).to(torch.bfloat16)
    gshape = (batch, heads, length) if per_head else (batch, length)
    lg = F.logsigmoid(gate_mean + gate_std * torch.randn(gshape, generator=g))
    dy = torch.randn(shape, generator=g).to(torch.bfloat16)
    return fq, fk, v, lg, dy


def rope_tables(length, dim, theta=500000.0):
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    ang = torch.outer(torch.arange(length, dtype=torch.float64), inv)
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()


def baseline_swa_inputs(batch, heads, length, dim, sinks=4, seed=0):
    """q, k, v = N(0,1); RoPE (theta 500000, rotate_half) on
    q and k in fp32, then bf16; meta = N(0,1) fp32 [sinks]; dO = N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    shape = (batch, heads, length, dim)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    cos, sin = rope_tables(length, dim)
    half = dim // 2

    def rope(x):
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return (x.double() * cos + rot.double() * sin).float()
    q, k = rope(q), rope(k)
    meta = torch.randn(sinks, generator=g)
    dy = torch.randn(shape, generator=g).to(torch.bfloat16)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), meta, dy


def gla_flops(batch, heads, length, nf, nd, chunk=64, backward=False):
    """Algorithmic flops per call: fwd 4FD + 2CF + 2CD per token and head,
    fwd+bwd 12FD + 8CF + 6CD (the reference's algorithm)."""
    per = (12 * nf * nd + 8 * chunk * nf + 6 * chunk * nd) if backward else \
        (4 * nf * nd + 2 * chunk * nf + 2 * chunk * nd)
    return batch * heads * length * per


def swa_weff(length, window):
    return sum(min(i + 1, window) for i in range(length)) / length


def swa_flops(batch, heads, length, dim, window, backward=False):
    return (14 if backward else 4) * dim * swa_weff(length, window) * batch * heads * length


def seconds(fn):  # pragma: no cover - helper for manual timing
    import time
    t = time.perf_counter()
    fn()
    return time.perf_counter() - t


__all__ = [n for n in dir() if not n.startswith("_")] + ["math"]
