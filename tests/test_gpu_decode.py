"""The recurrent decode path of GLA (the form of the reference's
tests/test_lizard.py:41-52): ``gla_prefill`` returns the chunked forward's
output and the state after the last token; ``gla_decode_step`` advances it
one token at a time.  Checked against the oracle's recurrent form with its
state (``gla_recurrent_state``, pinned in tests/test_oracle.py)."""
import pytest
import torch

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import OUT_TOL, baseline_gla_inputs, gla_inputs, max_rel

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
