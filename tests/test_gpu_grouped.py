"""Grouped-query operands: the GLA and SWA kernels given k-side tensors with
kv_heads < heads read each query head's operands from its kv head
(head h -> h // (heads // kv_heads)).  That must be exactly the computation on
the operands the reference's layer builds with repeat_interleave
(src/lizard_attention.py:73-76): bitwise equal outputs and gradients."""
import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels

pytestmark = pytest.mark.gpu


def _expand(t, group):
    return t.repeat_interleave(group, dim=1).contiguous()


@pytest.mark.parametrize("b, heads, kv, length, nf, nd, per_head", [
    (2, 8, 2, 300, 64, 64, True),      # segmented walks (B*H small)
    (2, 8, 2, 300, 64, 64, False),     # segmented, per-token gate: records per kv head
    (1, 32, 8, 777, 256, 64, False),   # the layer's wide features, two segments per walk
    # per-token gate, F = 128: the kv-head records' state pass splits its feature
    # rows over two workgroups (120 segments), the expanded one does not (480)
    (1, 32, 8, 2048, 128, 128, False),
    # B*H fills the GPU: one segment per (b, h), whose dq and dkv walks run in
    # one workgroup (512 of them, two rounds), grouped (XCD-mapped) and expanded
    (16, 32, 8, 130, 128, 128, True),
    # 5 segments per (b, h) and 500 dkv-walk workgroups at one per CU: the
    # dkv walk runs in rounds and takes its blocks in reverse per XCD
    (2, 50, 10, 600, 64, 64, False),
    # at most 4 segments: the walks fold the segment records (kv-head records
    # with a per-token gate; two segments per eight-wave walk at F = 256)
    (2, 64, 16, 500, 256, 64, False), (2, 64, 16, 500, 256, 64, True),
    (2, 64, 16, 461, 128, 128, False),
    (2, 64, 16, 300, 256, 128, True),   # two D tiles, each folding its records
    # past the walks' sizes, both gate kinds: two D tiles (the fused bf16 layer
    # at head_dim 128 x 128 features), two F tiles (summed raw numerators),
    # and ragged F and D tiles
    (1, 8, 2, 300, 256, 128, False), (1, 8, 2, 300, 256, 128, True),
    (1, 4, 2, 200, 512, 64, True), (1, 4, 2, 200, 512, 64, False),
    (1, 4, 2, 150, 300, 200, True), (2, 6, 3, 150, 300, 200, False),
])
def test_gla_grouped_kv_equals_expanded(b, heads, kv, length, nf, nd, per_head):
    g = torch.Generator().manual_seed(nf + length)
    group = heads // kv
    fq = F.softplus(torch.randn(b, heads, length, nf, generator=g)).bfloat16().cuda()
    fk = F.softplus(torch.randn(b, kv, length, nf, generator=g)).bfloat16().cuda()
    v = torch.randn(b, kv, length, nd, generator=g).bfloat16().cuda()
    lg = F.logsigmoid(2 + torch.randn(*((b, heads, length) if per_head else (b, length)),
                                      generator=g)).cuda()
    dy = torch.randn(b, heads, length, nd, generator=g).bfloat16().cuda()
    y1, st1 = kernels.gla_forward(fq, fk, v, lg, keep_state=True)
    fke, ve = _expand(fk, group), _expand(v, group)
    y2, st2 = kernels.gla_forward(fq, fke, ve, lg, keep_state=True)
    g1 = kernels.gla_backward(fq, fk, v, lg, dy, st1, torch.bfloat16)
    g2 = kernels.gla_backward(fq, fke, ve, lg, dy, st2, torch.bfloat16)
    # without the forward's segment records the backward recomputes them itself
    g3 = kernels.gla_backward(fq, fk, v, lg, dy, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert y1.shape == (b, heads, length, nd) and torch.equal(y1, y2)
    for name, a, r, c in zip(("dfq", "dfk", "dv", "dlog_gamma"), g1, g2, g3):
        assert a.shape == r.shape and torch.equal(a, r) and torch.equal(a, c), name


def test_gla_prefill_state_with_expanded_operands_matches_walk():
    # the recurrent state after a prefill does not depend on how the operands
    # are laid out either (prefill takes per-head operands)
    g = torch.Generator().manual_seed(11)
    fq = F.softplus(torch.randn(1, 4, 200, 64, generator=g)).bfloat16().cuda()
    fk = F.softplus(torch.randn(1, 2, 200, 64, generator=g)).bfloat16().cuda()
    v = torch.randn(1, 2, 200, 64, generator=g).bfloat16().cuda()
    lg = F.logsigmoid(3 + torch.randn(1, 200, generator=g)).cuda()
    y1, _ = kernels.gla_forward(fq, fk, v, lg, keep_state=False)
    y2, _ = kernels.gla_prefill(fq, _expand(fk, 2), _expand(v, 2), lg)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("b, heads, kv, length, d, window, n_meta", [
    (2, 8, 2, 300, 64, 64, 4), (1, 32, 8, 2048, 64, 64, 4), (1, 6, 3, 97, 128, 16, 0)])
def test_swa_grouped_kv_equals_expanded(b, heads, kv, length, d, window, n_meta):
    g = torch.Generator().manual_seed(d + length)
    group = heads // kv
    q = torch.randn(b, heads, length, d, generator=g).bfloat16().cuda()
    k = torch.randn(b, kv, length, d, generator=g).bfloat16().cuda()
    v = torch.randn(b, kv, length, d, generator=g).bfloat16().cuda()
    meta = torch.randn(n_meta, generator=g).cuda()
    dy = torch.randn(b, heads, length, d, generator=g).bfloat16().cuda()
    y1, lse1 = kernels.swa_forward(q, k, v, meta, window)
    ke, ve = _expand(k, group), _expand(v, group)
    y2, lse2 = kernels.swa_forward(q, ke, ve, meta, window)
    g1 = kernels.swa_backward(q, k, v, meta, lse1, dy, window, torch.bfloat16)
    g2 = kernels.swa_backward(q, ke, ve, meta, lse2, dy, window, torch.bfloat16)
    torch.cuda.synchronize()
    assert y1.shape == (b, heads, length, d) and torch.equal(y1, y2) and torch.equal(lse1, lse2)
    for name, a, r in zip(("dq", "dk", "dv", "dmeta"), g1, g2):
        assert a.shape == r.shape and torch.equal(a, r), name
