"""The recurrent decode path of GLA (the form of the reference's
tests/test_lizard.py:41-52): ``gla_prefill`` returns the chunked forward's
output and the state after the last token; ``gla_decode_step`` advances it
one token at a time.  Checked against the oracle's recurrent form with its
state (``gla_recurrent_state``, pinned in tests/test_oracle.py).

The SWA decode step (one query against a ring-buffered window cache) is
checked against the oracle's dense sliding-window softmax (``awa``) row by
row, and the layer's ``prefill`` + ``step`` against the layer's own forward
over the whole sequence and the oracle's dense layer (``lizard_layer``)."""
import pytest
import torch

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import (OUT_TOL, baseline_gla_inputs, gla_inputs, max_rel, norm_rel,
                           swa_inputs)
from tests.test_gpu_layer import random_layer
from tests.test_layer import tiny_rope

pytestmark = pytest.mark.gpu


def oracle_state(fq, fk, v, lg):
    """Outputs and final state of the recurrent form in fp64 on the bf16 inputs."""
    gamma = torch.exp(lg.double())
    return lo.gla_recurrent_state(fq.double(), fk.double(), v.double(), gamma)


@pytest.mark.parametrize("length, per_head, nf, nd", [
    (150, False, 24, 20), (300, True, 64, 64), (1, False, 32, 32), (129, True, 256, 64)])
def test_prefill_state_matches_recurrent_form(length, per_head, nf, nd):
    fq, fk, v, z = gla_inputs(length, gates=(3,) if per_head else (), features=nf, dim=nd)
    lg = torch.nn.functional.logsigmoid(z)
    y, state = kernels.gla_prefill(fq.cuda(), fk.cuda(), v.cuda(), lg.cuda())
    with torch.no_grad():
        y_ref = kernels.gla(fq.cuda(), fk.cuda(), v.cuda(), lg.cuda())
    out, S, zs = oracle_state(fq, fk, v, lg)
    S_k, z_k = kernels.split_state(state, nf, nd)
    torch.cuda.synchronize()
    errs = {"y": max_rel(y, out), "S": max_rel(S_k, S), "z": max_rel(z_k, zs)}
    print(f"[parity] prefill L={length} F={nf} D={nd} per_head={per_head}: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert torch.equal(y, y_ref)   # the same forward kernel
    assert max(errs.values()) <= OUT_TOL, errs


@pytest.mark.parametrize("prefix, steps, per_head, nf, nd", [
    (100, 40, False, 24, 20), (0, 30, True, 24, 20), (64, 65, False, 24, 20),
    # vector decode kernel (F % 4 == 0, D a power of two): 1, 2, 4 and 8 rows per thread
    (70, 20, True, 32, 32), (30, 12, False, 64, 128), (50, 10, True, 128, 64),
    (20, 8, False, 256, 64), (9, 5, True, 128, 128), (5, 3, False, 8, 4),
    (40, 6, False, 64, 64)])
def test_decode_steps_continue_the_sequence(prefix, steps, per_head, nf, nd):
    """Prefill on the first tokens, then one decode step per token: every
    step's output is the whole sequence's output at that position, and the
    final state is the whole sequence's."""
    n = prefix + steps
    fq, fk, v, z = gla_inputs(n, gates=(3,) if per_head else (), features=nf, dim=nd, seed=3)
    lg = torch.nn.functional.logsigmoid(z)
    b, h = fq.shape[:2]
    dev = [t.cuda() for t in (fq, fk, v, lg)]
    if prefix:
        _, state = kernels.gla_prefill(*(t[..., :prefix, :] for t in dev[:3]),
                                       dev[3][..., :prefix])
    else:
        state = kernels.new_state(b, h, nf, nd, "cuda")
    ys = [kernels.gla_decode_step(dev[0][:, :, i], dev[1][:, :, i], dev[2][:, :, i],
                                  dev[3][..., i], state) for i in range(prefix, n)]
    out, S, zs = oracle_state(fq, fk, v, lg)
    S_k, z_k = kernels.split_state(state, nf, nd)
    torch.cuda.synchronize()
    errs = {"y": max_rel(torch.stack(ys, dim=2), out[:, :, prefix:]),
            "S": max_rel(S_k, S), "z": max_rel(z_k, zs)}
    print(f"[parity] decode prefix={prefix} steps={steps} per_head={per_head} F={nf} D={nd}: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(y.dtype == torch.bfloat16 for y in ys)
    assert max(errs.values()) <= OUT_TOL, errs


def test_decode_at_the_config5_shape():
    """One decode step at the config-5 attention shape (B=4, 32 heads,
    F=256, D=64) after a 1000-token prefill with BASELINE's distributions."""
    fq, fk, v, lg, _ = baseline_gla_inputs(4, 32, 1001, 64, seed=4)
    fq, fk = torch.cat([fq, fq], -1), torch.cat([fk, fk], -1)   # F = 256
    dev = [t.cuda() for t in (fq, fk, v, lg)]
    y_full = kernels.gla(*dev)
    _, state = kernels.gla_prefill(*(t[..., :1000, :] for t in dev[:3]), dev[3][..., :1000])
    y = kernels.gla_decode_step(dev[0][:, :, 1000], dev[1][:, :, 1000], dev[2][:, :, 1000],
                                dev[3][:, 1000], state)
    torch.cuda.synchronize()
    err = max_rel(y, y_full[:, :, 1000])
    print(f"[parity] decode config5 shape vs chunked forward: {err:.2e}", flush=True)
    assert err <= OUT_TOL


def test_decode_rejects_bad_shapes():
    x = torch.zeros(2, 3, 8, device="cuda")
    with pytest.raises(ValueError):
        kernels.gla_decode_step(x, x, x, torch.zeros(2, 3, 4, device="cuda"),
                                kernels.new_state(2, 3, 8, 8, "cuda"))
    with pytest.raises(ValueError):
        kernels.gla_decode_step(x, x, x, torch.zeros(2, device="cuda"),
                                torch.zeros(2, 3, 10, device="cuda"))


def test_decode_with_kv_heads_equals_expanded_heads():
    """fk, v given per kv head: bitwise the decode of the expanded operands."""
    fq, fk, v, z = gla_inputs(12, batch=2, heads=4, features=32, dim=32, seed=8)
    lg = torch.nn.functional.logsigmoid(z).cuda()
    fq, fk, v = fq.cuda(), fk[:, :2].cuda(), v[:, :2].cuda()
    s1 = kernels.new_state(2, 4, 32, 32, "cuda")
    s2 = kernels.new_state(2, 4, 32, 32, "cuda")
    for i in range(12):
        y1 = kernels.gla_decode_step(fq[:, :, i], fk[:, :, i], v[:, :, i], lg[:, i], s1)
        y2 = kernels.gla_decode_step(fq[:, :, i], fk[:, :, i].repeat_interleave(2, 1),
                                     v[:, :, i].repeat_interleave(2, 1), lg[:, i], s2)
        assert torch.equal(y1, y2), i
    torch.cuda.synchronize()
    assert torch.equal(s1, s2)


@pytest.mark.parametrize("b, heads, kv, length, d, window, n_meta", [
    (2, 4, 2, 50, 64, 16, 4),      # window wraps the ring buffer three times
    (1, 2, 2, 300, 128, 128, 0),   # no sinks, the layer's window
    (1, 3, 1, 20, 32, 64, 4),      # window longer than the sequence
    (1, 2, 1, 40, 20, 8, 2),       # head dim not a multiple of 8
    (1, 2, 2, 70, 64, 1, 4),       # window 1: the current key only
])
def test_swa_decode_matches_oracle_rows(b, heads, kv, length, d, window, n_meta):
    """Decode each position against a ring cache filled one position at a
    time: every row is the dense oracle's row, and matches the forward
    kernel's row."""
    q, k, v, meta = swa_inputs(length, batch=b, heads=heads, dim=d, sinks=n_meta, seed=d)
    k, v = k[:, :kv], v[:, :kv]
    group = heads // kv
    expected = lo.swa_kernel_api(q, k.repeat_interleave(group, 1), v.repeat_interleave(group, 1),
                                 meta, window, torch.float64)
    qd, kd, vd, md = q.cuda(), k.cuda(), v.cuda(), meta.cuda()
    y_fwd, _ = kernels.swa_forward(qd, kd.contiguous(), vd.contiguous(), md, window)
    kc = torch.zeros(b, kv, window, d, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    rows = []
    for p in range(length):
        kc[:, :, p % window] = kd[:, :, p]
        vc[:, :, p % window] = vd[:, :, p]
        rows.append(kernels.swa_decode_step(qd[:, :, p], kc, vc, md, p))
    y = torch.stack(rows, dim=2)
    torch.cuda.synchronize()
    errs = {"oracle": max_rel(y, expected), "forward": max_rel(y, y_fwd)}
    print(f"[parity] swa decode B={b} H={heads}/{kv} L={length} d={d} W={window} "
          f"sinks={n_meta}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert y.dtype == torch.bfloat16
    assert max(errs.values()) <= OUT_TOL, errs


def test_swa_decode_rejects_bad_arguments():
    q = torch.zeros(1, 4, 64, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(1, 3, 16, 64, device="cuda", dtype=torch.bfloat16)   # 3 does not divide 4
    meta = torch.zeros(4, device="cuda")
    with pytest.raises(ValueError):
        kernels.swa_decode_step(q, kc, kc, meta, 0)
    kc = torch.zeros(1, 2, 16, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        kernels.swa_decode_step(q, kc, kc, meta, -1)
    big = torch.zeros(1, 2, kernels.SWA_DECODE_MAX_WINDOW + 1, 64, device="cuda",
                      dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        kernels.swa_decode_step(q, big, big, meta, 0)


@pytest.mark.parametrize("dtype, prefix, steps", [
    (torch.float32, 37, 12), (torch.float32, 0, 20), (torch.bfloat16, 5, 3),
    (torch.bfloat16, 70, 9)])
def test_layer_prefill_and_steps_continue_the_forward(dtype, prefix, steps):
    """prefill on the first tokens, then one step per token: each step's
    output is the forward's output at that position over the whole sequence
    (window 16, so the ring buffer wraps), and the dense oracle layer's (fp64
    on the same parameters).  fp32: the north-star bar on the max error;
    bf16: the bf16 layer bars on the relative norm (1e-2 against our own
    forward, the reference's 2e-2 against the oracle, tests/test_lizard.py:244-253)."""
    layer = random_layer(dtype, seed=5)
    params = {n: p.detach().double() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    n, b = prefix + steps, 2
    x = torch.randn(b, n, 128, generator=torch.Generator().manual_seed(6)).to(dtype)
    cos, sin = (t.to(dtype) for t in tiny_rope(n, batch=b, dtype=torch.float32))
    xd, cd, sd = x.cuda(), cos.cuda(), sin.cuda()
    with torch.no_grad():
        full, _ = layer(xd, (cd, sd))
    expected = lo.lizard_layer(params, x.double(), cos.double(), sin.double(), 4, 2, 16)
    if prefix:
        out, cache = layer.prefill(xd[:, :prefix], (cd[:, :prefix], sd[:, :prefix]))
        assert torch.equal(out, full[:, :prefix])   # the same forward kernels
    else:
        cache = layer.new_cache(b)
    outs = [layer.step(xd[:, p:p + 1], (cd[:, p:p + 1], sd[:, p:p + 1]), cache)
            for p in range(prefix, n)]
    y = torch.cat(outs, dim=1)
    torch.cuda.synchronize()
    errs = {"forward_max": max_rel(y, full[:, prefix:]),
            "forward_norm": norm_rel(y, full[:, prefix:]),
            "oracle_max": max_rel(y, expected[:, prefix:]),
            "oracle_norm": norm_rel(y, expected[:, prefix:])}
    print(f"[parity] layer decode {dtype} prefix={prefix} steps={steps}: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert y.dtype == dtype and cache.pos == n
    if dtype == torch.float32:
        assert errs["forward_max"] <= OUT_TOL and errs["oracle_max"] <= OUT_TOL, errs
    else:
        assert errs["forward_norm"] < 1e-2 and errs["oracle_norm"] < 2e-2, errs
