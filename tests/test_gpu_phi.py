"""The GLA forward that forms fq inside its walk (lz_gla_fwd_phi): the
Hedgehog map of q (src/lizard_attention.py:9-11) computed chunk by chunk
from the q projection rows and phi_q instead of read from memory.  Checked
against the same walk fed the prologue's fq, against the fp64 oracle, and as
the layer's forward without autograd and prefill at config 5's shape."""
import types

import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels
from lizard_reproduction_amd import layer as hip_layer
from oracle import lizard_oracle as lo
from tests.helpers import OUT_TOL, max_rel, norm_rel

pytestmark = pytest.mark.gpu


def _operands(b, h, kv, length, per_head, seed):
    g = torch.Generator().manual_seed(seed)
    qp = torch.randn(b, length, h * 64, generator=g).bfloat16()
    kp = torch.randn(b, length, kv * 64, generator=g).bfloat16()
    vp = torch.randn(b, length, kv * 64, generator=g).bfloat16()
    wq = (0.15 * torch.randn(128, 64, generator=g)).bfloat16()
    wk = (0.15 * torch.randn(128, 64, generator=g)).bfloat16()
    z = 2 * torch.randn(*((b, h, length) if per_head else (b, length)), generator=g) + 2
    cos, sin = (t.bfloat16() for t in lo.rope_cos_sin(length, 64))
    return qp, kp, vp, wq, wk, z, cos, sin


@pytest.mark.parametrize("b, h, kv, length, per_head", [
    (1, 32, 8, 4096, False),   # config 5's layer shape, one batch row (segmented walks)
    (2, 4, 2, 300, True),      # ragged L, per-head gate
    (16, 32, 32, 130, False),  # B*H fills the GPU: one walk per (b, h)
    (1, 2, 1, 1, True),        # a single token
])
def test_gla_forward_phi_matches_prologue_fq(b, h, kv, length, per_head):
    """y and the final state against the walk fed the prologue's fq (the same
    bf16 product x W^T; the softmax sums meet in another order, so fq may
    differ in its last bit), and y against the fp64 oracle on exact
    hedgehog(q) features."""
    qp, kp, vp, wq, wk, z, cos, sin = (t.cuda() for t in _operands(b, h, kv, length, per_head,
                                                                   length + h))
    fq, fk, qr, kr, v, _ = hip_layer.prologue_forward(qp, kp, vp, wq, wk, cos, sin, h, kv)
    y_ref, st_ref = kernels.gla_prefill(fq, fk, v, z, gate_logit=True)
    _, fk2, _, _, v2, _ = hip_layer.prologue_forward(qp, kp, vp, wq, wk, cos, sin, h, kv,
                                                     with_fq=False)
    y, st = kernels.gla_forward_phi(qp, wq, fk2, v2, z, h, gate_logit=True, final_state=True)
    y_nostate, none = kernels.gla_forward_phi(qp, wq, fk2, v2, z, h, gate_logit=True)
    torch.cuda.synchronize()
    assert none is None and torch.equal(y, y_nostate)
    assert torch.equal(fk, fk2) and torch.equal(v, v2)
    # the oracle: exact features of the bf16 q rows, the kernels' bf16 fk and v
    rows = (0, b - 1)
    q64 = qp.double().cpu().view(b, length, h, 64).transpose(1, 2)[list(rows)]
    fq64 = lo.hedgehog(q64, wq.double().cpu())
    group = h // kv
    ref = lo.gla_chunked(fq64, fk.double().cpu()[list(rows)].repeat_interleave(group, 1),
                         v.double().cpu()[list(rows)].repeat_interleave(group, 1),
                         F.logsigmoid(z.double().cpu()[list(rows)]), 64)
    errs = {"y_vs_prologue_fq": max_rel(y, y_ref), "state_vs_prologue_fq": max_rel(st, st_ref),
            "y_oracle": max_rel(y[list(rows)], ref)}
    print(f"[parity] gla phi b={b} h={h}/{kv} L={length} per_head={per_head}: " +
          " ".join(f"{k}={e:.2e}" for k, e in errs.items()), flush=True)
    assert errs["y_oracle"] <= OUT_TOL, errs
    assert errs["y_vs_prologue_fq"] <= 8e-3 and errs["state_vs_prologue_fq"] <= 1e-3, errs


def _config5_layer(length=4096):
    cfg = types.SimpleNamespace(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8)
    torch.manual_seed(0)
    layer = hip_layer.LizardAttention(cfg, 0, window=64, num_meta=4, feature_dim=128)
    with torch.no_grad():
        layer.phi_q.weight.normal_(0, 0.3)
        layer.phi_k.weight.normal_(0, 0.3)
        layer.W_gamma.weight.normal_(0, 0.05)
        layer.meta_tokens.normal_(0, 1)
        layer.alpha_blend.fill_(0.8)
    layer = layer.bfloat16()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, length, 2048, generator=g).bfloat16()
    cos, sin = (t[None].expand(1, length, 64).bfloat16() for t in lo.rope_cos_sin(length, 64))
    return layer, x, cos, sin


def test_config5_layer_inference_forms_fq_in_the_walk():
    """Config 5's layer (bf16, B=1 slice of L=4096) without autograd takes the
    walk that forms fq itself: its output against the same layer's autograd
    forward (prologue fq), the exact oracle layer (the reference's bf16
    layer bar, 2e-2 relative norm, tests/test_lizard.py:244-253) and the
    bf16 rounding model of the layer (north-star output bar)."""
    layer, x, cos, sin = _config5_layer()
    params = {n: p.detach().double() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    xc, rope = x.cuda(), (cos.cuda(), sin.cuda())
    with torch.no_grad():
        y_phi = layer(xc, rope)[0]
    y_core = layer(xc.requires_grad_(), rope)[0].detach()
    torch.cuda.synchronize()
    with torch.no_grad():
        exact = lo.lizard_layer_rounded(params, x.double(), cos.double(), sin.double(), 32, 8,
                                        64, rounded=False)
        model = lo.lizard_layer_rounded(params, x.double(), cos.double(), sin.double(), 32, 8,
                                        64, rounded=True, bf16_layer=True)
    errs = {"vs_autograd_forward": max_rel(y_phi, y_core), "norm_vs_exact": norm_rel(y_phi, exact),
            "vs_rounding_model": max_rel(y_phi, model)}
    print("[parity] config5 bf16 layer inference (fq in the walk): " +
          " ".join(f"{k}={e:.2e}" for k, e in errs.items()), flush=True)
    assert y_phi.dtype == torch.bfloat16
    assert errs["norm_vs_exact"] < 2e-2 and errs["vs_rounding_model"] <= OUT_TOL, errs
    assert errs["vs_autograd_forward"] <= 1e-2, errs


def test_config5_layer_prefill_then_steps():
    """prefill (fq in the walk, and the state after the prompt) on 1000
    tokens, then 3 decode steps, against the forward over all 1003 tokens."""
    layer, x, cos, sin = _config5_layer(1003)
    layer = layer.cuda()
    xc, cc, sc = x.cuda(), cos.cuda(), sin.cuda()
    with torch.no_grad():
        full = layer(xc, (cc, sc))[0]
        out, cache = layer.prefill(xc[:, :1000], (cc[:, :1000], sc[:, :1000]))
        steps = [layer.step(xc[:, i:i + 1], (cc[:, i:i + 1], sc[:, i:i + 1]), cache)
                 for i in range(1000, 1003)]
    torch.cuda.synchronize()
    errs = {"prefill": max_rel(out, full[:, :1000]),
            "steps": max_rel(torch.cat(steps, 1), full[:, 1000:])}
    print("[parity] config5 bf16 layer prefill+steps: " +
          " ".join(f"{k}={e:.2e}" for k, e in errs.items()), flush=True)
    assert errs["prefill"] == 0.0, errs          # the same path as the forward
    assert errs["steps"] <= OUT_TOL, errs
