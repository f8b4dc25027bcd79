"""The GLA kernels' logit gate mode (LZ_GATE_LOGIT): the gate buffer holds the
logit z and the kernels form log_gamma = logsigmoid(z) themselves, returning
the gradient of z -- the layer's F.logsigmoid (src/lizard_attention.py:92)
fused into the gate path.  Checked against the oracle with autograd through
logsigmoid, and against the same kernels fed torch's logsigmoid(z)."""
import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import GRAD_TOL, OUT_TOL, max_rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b, h, kv, length, nf, nd, per_head", [
    (1, 4, 4, 300, 64, 64, False),     # segmented walks, per-token gate (gate launch)
    (2, 8, 2, 200, 64, 32, True),      # segmented, per-head gate, grouped kv heads
    (4, 128, 128, 130, 64, 64, True),  # one segment per (b, h): the dkv walk writes dz
    (1, 2, 1, 150, 300, 200, False),   # tiled sizes past the walks'
    (1, 3, 3, 1, 32, 32, True),        # a single token
])
def test_gla_gate_logit_matches_oracle(b, h, kv, length, nf, nd, per_head):
    g = torch.Generator().manual_seed(length + nf)
    fq = F.softplus(torch.randn(b, h, length, nf, generator=g)).bfloat16()
    fk = F.softplus(torch.randn(b, kv, length, nf, generator=g)).bfloat16()
    v = torch.randn(b, kv, length, nd, generator=g).bfloat16()
    # logits both ways of 0 and large enough for log1p(e^-|z|) to underflow
    z = 3 * torch.randn(*((b, h, length) if per_head else (b, length)), generator=g) + 1
    z.view(-1)[:4] = torch.tensor([-30.0, 30.0, 0.0, 90.0])[: z.numel()]
    dy = torch.randn(b, h, length, nd, generator=g).bfloat16()
    dev = [t.cuda() for t in (fq, fk, v, z, dy)]
    y, st = kernels.gla_forward(*dev[:4], keep_state=True, gate_logit=True)
    dfq, dfk, dv, dz = kernels.gla_backward(*dev[:4], dev[4], st, torch.float32, gate_logit=True)
    lg = F.logsigmoid(dev[3])
    y2, st2 = kernels.gla_forward(*dev[:3], lg, keep_state=True)
    g2 = kernels.gla_backward(*dev[:3], lg, dev[4], st2, torch.float32)
    torch.cuda.synchronize()
    # the oracle, with autograd through logsigmoid to z
    group = h // kv
    leaves = [t.double().requires_grad_() for t in (fq, fk.repeat_interleave(group, 1),
                                                    v.repeat_interleave(group, 1), z)]
    ref = lo.gla_kernel_api(*leaves[:3], F.logsigmoid(leaves[3]), dtype=torch.float64)
    ref.backward(dy.double())
    errs = {"y": max_rel(y, ref), "dfq": max_rel(dfq, leaves[0].grad),
            "dz": max_rel(dz, leaves[3].grad),
            "y_vs_lg": max_rel(y, y2), "dz_vs_dlg": max_rel(dz, g2[3] * torch.sigmoid(-dev[3]))}
    print(f"[parity] gate logit b={b} h={h}/{kv} L={length} F={nf} D={nd} per_head={per_head}: "
          + " ".join(f"{k}={e:.2e}" for k, e in errs.items()), flush=True)
    assert dz.shape == z.shape and dz.dtype == torch.float32
    assert errs["y"] <= OUT_TOL and errs["dfq"] <= GRAD_TOL and errs["dz"] <= GRAD_TOL, errs
    # the two kernel paths differ only by the fp32 rounding of logsigmoid, which
    # can move a bf16 output by an ulp (2^-8 of the max-abs): two ulps allowed
    assert errs["y_vs_lg"] <= 2 * 2 ** -8 and errs["dz_vs_dlg"] <= 1e-3, errs
    assert torch.isfinite(dz).all()


@pytest.mark.parametrize("per_head", [False, True])
def test_gla_prefill_and_decode_take_the_gate_logit(per_head):
    """Prefill on 100 tokens, then 5 decode steps, with the gate given as
    logits, against the same calls given torch's logsigmoid of them."""
    g = torch.Generator().manual_seed(7)
    b, h, n, nf, nd = 2, 4, 105, 64, 32
    fq = F.softplus(torch.randn(b, h, n, nf, generator=g)).bfloat16().cuda()
    fk = F.softplus(torch.randn(b, h, n, nf, generator=g)).bfloat16().cuda()
    v = torch.randn(b, h, n, nd, generator=g).bfloat16().cuda()
    z = (2 * torch.randn(*((b, h, n) if per_head else (b, n)), generator=g) + 2).cuda()
    lg = F.logsigmoid(z)
    outs = []
    for gate, logit in ((z, True), (lg, False)):
        y, state = kernels.gla_prefill(fq[:, :, :100], fk[:, :, :100], v[:, :, :100],
                                       gate[..., :100].contiguous(), gate_logit=logit)
        steps = [kernels.gla_decode_step(fq[:, :, i], fk[:, :, i], v[:, :, i],
                                         gate[..., i].contiguous(), state, gate_logit=logit)
                 for i in range(100, n)]
        outs.append((y, torch.stack(steps, 2), state))
    torch.cuda.synchronize()
    errs = [max_rel(a, r) for a, r in zip(*outs)]
    print(f"[parity] gate logit prefill/decode per_head={per_head}: y={errs[0]:.2e} "
          f"steps={errs[1]:.2e} state={errs[2]:.2e}", flush=True)
    assert max(errs) <= 2 * 2 ** -8, errs
