"""Whole-layer parity of the HIP LizardAttention against the oracle's dense
layer, output and every parameter gradient (the reference's
tests/test_kernels.py:137-156), and of a small Llama with every attention
block swapped."""
import pytest
import torch
import torch.nn as nn
from transformers import LlamaForCausalLM

from lizard_reproduction_amd import layer as hip_layer
from oracle import lizard_oracle as lo
from tests.helpers import GRAD_TOL, OUT_TOL, max_rel, norm_rel, ref_close
from tests.test_layer import tiny_config, tiny_rope

pytestmark = pytest.mark.gpu


def random_layer(dtype, seed=0, window=16, feature_dim=8):
    torch.manual_seed(seed)
    layer = hip_layer.LizardAttention(tiny_config(), 0, window=window, feature_dim=feature_dim)
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.3)
    return layer.to(dtype)


class OracleAttention(nn.Module):
    """The oracle's dense layer behind the layer's module interface, with
    its own copies of a LizardAttention's parameters (CPU)."""

    def __init__(self, layer):
        super().__init__()
        self.heads, self.kv_heads, self.window = layer.heads, layer.kv_heads, layer.window
        self.params = nn.ParameterDict({n.replace(".", "__"): nn.Parameter(p.detach().cpu().clone())
                                        for n, p in layer.named_parameters()})

    def forward(self, hidden_states, position_embeddings, **kwargs):
        params = {n.replace("__", "."): p for n, p in self.params.items()}
        cos, sin = position_embeddings
        return lo.lizard_layer(params, hidden_states, cos, sin, self.heads, self.kv_heads,
                               self.window), None


def report(label, pairs):
    for k, (a, b) in pairs.items():
        assert a is not None and b is not None, k
    out = {k: max_rel(a, b) for k, (a, b) in pairs.items()}
    print(f"[parity] {label}: " + " ".join(f"{k}={v:.2e}" for k, v in out.items()), flush=True)
    return out


@pytest.mark.parametrize("length", [40, 130])
def test_layer_matches_oracle_layer(length):
    """fp32 layer (the reference's whole-layer test shape, L=40, plus a
    length that spans three GLA chunks); every parameter gradient and the
    input gradient within the north-star bars."""
    layer = random_layer(torch.float32)
    oracle = OracleAttention(layer)
    layer = layer.cuda()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, length, 128, generator=g)
    grad = torch.randn(2, length, 128, generator=g)
    rope = tiny_rope(length, batch=2, dtype=torch.float32)
    xg = x.detach().cuda().requires_grad_()
    y = layer(xg, tuple(t.cuda() for t in rope))[0]
    y.backward(grad.cuda())
    xc = x.detach().clone().requires_grad_()
    expected = oracle(xc, rope)[0]
    expected.backward(grad)
    torch.cuda.synchronize()
    pairs = {"out": (y, expected), "dx": (xg.grad, xc.grad)}
    for name, p in layer.named_parameters():
        pairs[name] = (p.grad, oracle.params[name.replace(".", "__")].grad)
    errs = report(f"layer L={length}", pairs)
    assert y.dtype == torch.float32
    assert errs["out"] <= OUT_TOL and norm_rel(y, expected) < 2 * OUT_TOL, errs
    for name, (a, b) in pairs.items():
        if name == "out":
            continue
        assert errs[name] <= GRAD_TOL, (name, errs)
        assert ref_close(a, b), (name, errs)


def test_bf16_layer_stays_bf16_and_close_to_oracle():
    """bf16 weights and activations (the config-5 dtype): the output stays
    bf16 and is within the reference's bf16 layer bar (2e-2 relative norm,
    tests/test_lizard.py:244-253) of the fp64 oracle on the same bf16
    parameters."""
    layer = random_layer(torch.bfloat16)
    params = {n: p.detach().double() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    x = torch.randn(2, 40, 128, generator=torch.Generator().manual_seed(2)).bfloat16()
    rope = tiny_rope(40, batch=2, dtype=torch.float32)
    with torch.no_grad():
        y = layer(x.cuda(), tuple(t.cuda().bfloat16() for t in rope))[0]
    expected = lo.lizard_layer(params, x.double(), rope[0].bfloat16().double(),
                               rope[1].bfloat16().double(), 4, 2, 16)
    print(f"[parity] bf16 layer: norm={norm_rel(y, expected):.2e} "
          f"max={max_rel(y, expected):.2e}", flush=True)
    assert y.dtype == torch.bfloat16
    assert norm_rel(y, expected) < 2e-2


def test_small_llama_with_lizard_blocks_matches_oracle_model():
    """A 2-block Llama (fp32) with every attention block swapped: logits and
    the gradients of every parameter of the model after a cross-entropy
    backward, HIP layers on the GPU vs oracle layers on the CPU."""
    torch.manual_seed(0)
    model = LlamaForCausalLM(tiny_config(layers=2))
    hip_layer.to_lizard(model, window=16, feature_dim=8)
    with torch.no_grad():
        for block in model.model.layers:
            for p in block.self_attn.parameters():
                if p.dim() < 2 or p.shape[0] == 1 or p.shape[1] == 32:
                    p.normal_(0, 0.3)   # lizard-only parameters away from their init
    cpu = LlamaForCausalLM(tiny_config(layers=2))
    cpu.load_state_dict({k: v for k, v in model.state_dict().items()
                         if "self_attn" not in k}, strict=False)
    for mine, theirs in zip(cpu.model.layers, model.model.layers):
        mine.self_attn = OracleAttention(theirs.self_attn)
    model = model.cuda()
    ids = torch.randint(0, 100, (2, 96), generator=torch.Generator().manual_seed(3))
    out = model(ids.cuda(), labels=ids.cuda())
    out.loss.backward()
    ref = cpu(ids, labels=ids)
    ref.loss.backward()
    torch.cuda.synchronize()
    pairs = {"logits": (out.logits, ref.logits)}
    cpu_params = dict(cpu.named_parameters())
    for name, p in model.named_parameters():
        if "self_attn" in name:
            block, rest = name.split(".self_attn.")
            theirs = cpu_params[f"{block}.self_attn.params.{rest.replace('.', '__')}"]
        else:
            theirs = cpu_params[name]
        pairs[name] = (p.grad, theirs.grad)
    errs = report("llama x2", pairs)
    assert abs(out.loss.item() - ref.loss.item()) < 1e-3 * abs(ref.loss.item())
    assert errs["logits"] <= OUT_TOL, errs
    for name, (a, b) in pairs.items():
        if name != "logits":
            assert errs[name] <= GRAD_TOL, (name, errs)


# -- the fused prologue and epilogue on their own ------------------------------

def prologue_reference(qp, kp, vp, wq, wk, cos, sin, heads, kv_heads):
    """The reference's ops between the projections and the kernels
    (src/lizard_attention.py:73-88), from the oracle's hedgehog and rope."""
    b, length, _ = qp.shape
    hd = qp.shape[-1] // heads

    def split(x, n):
        return x.view(b, length, n, hd).transpose(1, 2).repeat_interleave(heads // n, dim=1)
    q, k, v = split(qp, heads), split(kp, kv_heads), split(vp, kv_heads)
    c, s = ((t if t.dim() == 3 else t[None]) for t in (cos, sin))
    c, s = c.unsqueeze(1), s.unsqueeze(1)
    return (lo.hedgehog(q, wq), lo.hedgehog(k, wk), lo.rope(q, c, s), lo.rope(k, c, s), v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b, length, heads, kv, hd, f, batched", [
    (2, 40, 4, 2, 32, 8, True), (1, 300, 8, 2, 64, 128, False), (2, 77, 4, 4, 64, 64, True),
    (1, 129, 8, 1, 128, 64, True), (1, 50, 6, 3, 32, 12, False), (1, 33, 4, 2, 64, 100, True)])
def test_prologue_matches_reference_ops(dtype, b, length, heads, kv, hd, f, batched):
    """The fused prologue's outputs and, from the same upstream gradients
    (v's given as two parts, one per attention branch), every input
    gradient, against autograd through the reference's ops in fp64."""
    prologue_case(dtype, b, length, heads, kv, hd, f, batched)


@pytest.mark.parametrize("b, length, heads, kv, batched", [(1, 200, 8, 2, True),
                                                            (2, 70, 4, 4, False)])
def test_prologue_head_dim_128_with_128_features_bf16(b, length, heads, kv, batched):
    """head_dim 128 with feature_dim 128 (a head_dim-128 model at the
    reference's default feature_dim): bf16 arithmetic only."""
    prologue_case(torch.bfloat16, b, length, heads, kv, 128, 128, batched)


def prologue_case(dtype, b, length, heads, kv, hd, f, batched):
    g = torch.Generator().manual_seed(hd + f + length)
    qp = torch.randn(b, length, heads * hd, generator=g).to(dtype)
    kp = torch.randn(b, length, kv * hd, generator=g).to(dtype)
    vp = torch.randn(b, length, kv * hd, generator=g).to(dtype)
    wq = (0.3 * torch.randn(f, hd, generator=g)).to(dtype)
    wk = (0.3 * torch.randn(f, hd, generator=g)).to(dtype)
    cos, sin = lo.rope_cos_sin(length + 3, hd)
    cos, sin = cos[3:], sin[3:]
    if batched:
        cos, sin = cos[None].repeat(b, 1, 1), sin[None].repeat(b, 1, 1)
    cos, sin = cos.to(dtype), sin.to(dtype)
    # the prologue takes its upstream gradients in bf16: bf16-valued ones here
    ups = [torch.randn(b, heads, length, n, generator=g).bfloat16().float()
           for n in (2 * f, 2 * f, hd, hd, hd, hd)]
    *outs, saved = hip_layer.prologue_forward(*(t.cuda() for t in (qp, kp, vp, wq, wk, cos, sin)),
                                              heads, kv)
    grads = hip_layer.prologue_backward(saved, *(u.cuda() for u in ups))
    torch.cuda.synchronize()
    theirs = [t.detach().double().requires_grad_() for t in (qp, kp, vp, wq, wk)]
    refs = prologue_reference(*theirs, cos.double(), sin.double(), heads, kv)
    ref_ups = [u.double() for u in ups[:4]] + [(ups[4] + ups[5]).double()]
    torch.autograd.backward(refs, ref_ups)
    # the key-side operands are written once per kv head: the reference's
    # repeat_interleave copies them to the heads of each group, so its first
    # head of every group is the one to compare with
    group = heads // kv
    pairs = {n: (a, r if n in ("fq", "qr") else r[:, ::group])
             for n, a, r in zip(("fq", "fk", "qr", "kr", "v"), outs, refs)}
    for n in ("fk", "kr", "v"):
        assert pairs[n][0].shape[1] == kv, n
    for n, a, r in zip(("dq", "dk", "dv", "dwq", "dwk"), grads, theirs):
        pairs[n] = (a, r.grad)
    errs = report(f"prologue {dtype} b={b} L={length} H={heads}/{kv} hd={hd} f={f}", pairs)
    for n in ("fq", "fk", "qr", "kr", "v"):
        assert pairs[n][0].dtype == torch.bfloat16 and errs[n] <= OUT_TOL, (n, errs)
    for n in ("dq", "dk", "dv"):
        assert pairs[n][0].dtype == dtype, n
    for n in ("dq", "dk", "dv", "dwq", "dwk"):
        assert errs[n] <= GRAD_TOL, (n, errs)
    if dtype == torch.float32:
        # fp32 inputs: the split bf16 products keep the gradients near fp32 accuracy
        assert max(errs[n] for n in ("dq", "dk", "dv", "dwq", "dwk")) < 1e-4, errs


def test_prologue_is_deterministic():
    g = torch.Generator().manual_seed(5)
    args = [torch.randn(*s, generator=g).bfloat16().cuda()
            for s in ((2, 256, 512), (2, 256, 128), (2, 256, 128), (128, 64), (128, 64))]
    cos, sin = (t.bfloat16().cuda() for t in lo.rope_cos_sin(256, 64))
    ups = [torch.randn(2, 8, 256, n, generator=g).cuda() for n in (256, 256, 64, 64, 64)]
    runs = []
    for _ in range(2):
        *outs, saved = hip_layer.prologue_forward(*args, cos, sin, 8, 2)
        runs.append(outs + list(hip_layer.prologue_backward(saved, *ups)))
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_combine_matches_reference_ops(dtype):
    """The blend + transpose against the reference's torch ops
    (src/lizard_attention.py:94-97): bitwise equal output and branch
    gradients, alpha's gradient up to the order of its sum."""
    g = torch.Generator().manual_seed(7)
    yg = torch.randn(2, 4, 70, 32, generator=g).bfloat16()
    ys = torch.randn(2, 4, 70, 32, generator=g).bfloat16()
    alpha = torch.tensor(0.7)
    dout = torch.randn(2, 70, 128, generator=g).to(dtype)
    out = hip_layer.combine_forward(yg.cuda(), ys.cuda(), alpha.reshape(1).cuda(), dtype)
    dyg, dys, dalpha = hip_layer.combine_backward(dout.cuda(), ys.cuda(), alpha.reshape(1).cuda())
    leaves = [t.detach().clone().requires_grad_() for t in (yg, ys, alpha)]
    ref = (leaves[0].float() + leaves[2] * leaves[1].float()).to(dtype).transpose(1, 2).flatten(2)
    ref.backward(dout)
    assert out.dtype == dtype and torch.equal(out.cpu(), ref)
    assert torch.equal(dyg.cpu(), leaves[0].grad)
    assert torch.equal(dys.cpu(), leaves[1].grad)
    assert abs(dalpha.item() - leaves[2].grad.item()) <= 1e-5 * abs(leaves[2].grad.item())


def test_config5_layer_at_size_matches_banded_oracle_layer():
    """One LizardAttention at BASELINE config 5's shape -- hidden 2048, 32
    query / 8 kv heads, head_dim 64, feature_dim 128 (F = 256), window 64, 4
    sinks, RoPE theta 500000 -- on a B=1 slice of its L=4096 sequences, fp32
    parameters, against the long-L oracle layer (chunked GLA, banded SWA;
    pinned against the dense layer in tests/test_layer.py) in fp64: output,
    input gradient and every parameter gradient (the reference's whole-layer
    test, tests/test_kernels.py:137-156, at the model's size)."""
    import types
    cfg = types.SimpleNamespace(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8)
    torch.manual_seed(0)
    layer = hip_layer.LizardAttention(cfg, 0, window=64, num_meta=4, feature_dim=128)
    with torch.no_grad():
        layer.phi_q.weight.normal_(0, 0.3)
        layer.phi_k.weight.normal_(0, 0.3)
        layer.W_gamma.weight.normal_(0, 0.05)   # gates from ~0.1 to ~0.99
        layer.meta_tokens.normal_(0, 1)
        layer.alpha_blend.fill_(0.8)
    params = {n: p.detach().double().requires_grad_() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    batch, length = 1, 4096
    g = torch.Generator().manual_seed(5)
    x = torch.randn(batch, length, 2048, generator=g)
    gy = torch.randn(batch, length, 2048, generator=g)
    cos, sin = (t[None].expand(batch, length, 64) for t in lo.rope_cos_sin(length, 64))
    xg = x.cuda().requires_grad_()
    y = layer(xg, (cos.float().cuda(), sin.float().cuda()))[0]
    y.backward(gy.cuda())
    torch.cuda.synchronize()
    xc = x.double().requires_grad_()
    expected = lo.lizard_layer_banded(params, xc, cos, sin, 32, 8, 64)
    expected.backward(gy.double())
    pairs = {"out": (y, expected), "dx": (xg.grad, xc.grad)}
    for name, p in layer.named_parameters():
        pairs[name] = (p.grad, params[name].grad)
    errs = report("config5 layer B=1 L=4096", pairs)
    assert y.dtype == torch.float32
    assert errs["out"] <= OUT_TOL and norm_rel(y, expected) < OUT_TOL, errs
    for name, (a, b) in pairs.items():
        if name == "out":
            continue
        assert errs[name] <= GRAD_TOL, (name, errs)
        assert ref_close(a, b), (name, errs)


@pytest.mark.parametrize("hidden, heads, kv, feature_dim, length", [
    (256, 2, 1, 128, 70),   # head_dim 128, feature_dim 128, fp32: F = 256, D = 128 tiles
    (192, 2, 2, 24, 130),   # head_dim 96: not a fused-prologue head_dim
])
def test_layer_at_shapes_past_the_fused_prologue_matches_oracle(hidden, heads, kv, feature_dim,
                                                                 length):
    """fp32 layers whose shapes the fused prologue does not take run the
    reference's torch ops before the HIP GLA and SWA operators: output,
    input gradient and every parameter gradient against the dense oracle."""
    import types
    cfg = types.SimpleNamespace(hidden_size=hidden, num_attention_heads=heads,
                                num_key_value_heads=kv)
    torch.manual_seed(0)
    layer = hip_layer.LizardAttention(cfg, 0, window=16, feature_dim=feature_dim)
    hd = hidden // heads
    # the reference's layer tests draw phi ~ N(0, 0.3) at head_dim 32 (tiny
    # config); the feature logits q phi^T grow with sqrt(head_dim), so phi is
    # scaled to keep that logit scale (at 0.3 and head_dim 128 the Hedgehog
    # maps are nearly one-hot, and the gate weight's gradient -- a sum over
    # tokens that mostly cancels -- turns the kernels' 4-6e-3 error in
    # d log_gamma into 2.8e-2)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            kind = n.split(".")[0]
            std = 0.1 if kind in ("q_proj", "k_proj", "v_proj", "o_proj") else 0.3
            p.normal_(0, std * (32 / hd) ** 0.5 if kind in ("phi_q", "phi_k") else std)
    assert not hip_layer.prologue_supported(hd, feature_dim, bf16=False)
    oracle = OracleAttention(layer)
    layer = layer.cuda()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, length, hidden, generator=g)
    grad = torch.randn(2, length, hidden, generator=g)
    cos, sin = (t.float()[None].expand(2, length, hd) for t in lo.rope_cos_sin(length, hd))
    xg = x.cuda().requires_grad_()
    y = layer(xg, (cos.cuda(), sin.cuda()))[0]
    y.backward(grad.cuda())
    xc = x.clone().requires_grad_()
    expected = oracle(xc, (cos, sin))[0]
    expected.backward(grad)
    torch.cuda.synchronize()
    pairs = {"out": (y, expected), "dx": (xg.grad, xc.grad)}
    for name, p in layer.named_parameters():
        pairs[name] = (p.grad, oracle.params[name.replace(".", "__")].grad)
    errs = report(f"unfused layer hidden={hidden} hd={hd} f={feature_dim}", pairs)
    assert errs["out"] <= OUT_TOL, errs
    for name in pairs:
        if name != "out":
            assert errs[name] <= GRAD_TOL, (name, errs)


def _bf16_layer_case(layer, x, grad, cos, sin, heads, kv, window, label):
    """A bf16 layer forward+backward on the GPU against the fp64 oracle on
    the same bf16 parameters and inputs: the output within the reference's
    bf16 layer bar (2e-2 relative norm, tests/test_lizard.py:244-253) of the
    exact layer, and the output, input gradient and every parameter gradient
    within the north-star bar of the layer with the HIP path's bf16 rounding
    points (lo.lizard_layer_rounded, pinned to the exact layer in
    tests/test_layer.py)."""
    from tests.test_gpu_random_shapes import _oracle_layer_grads
    params = {n: p.detach().double() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    xg = x.cuda().requires_grad_()
    y = layer(xg, (cos.cuda(), sin.cuda()))[0]
    y.backward(grad.cuda())
    torch.cuda.synchronize()
    ours = {"out": y, "dx": xg.grad}
    ours.update({n: p.grad for n, p in layer.named_parameters()})
    model, exact = (_oracle_layer_grads(params, x, grad, cos, sin, heads, kv, window, rnd, True)
                    for rnd in (True, False))
    direct = report(label, {"rounding_model/" + n: (ours[n], model[n]) for n in ours})
    report(label, {n: (ours[n], exact[n]) for n in ours})
    err = norm_rel(y, exact["out"])
    print(f"[parity] {label}: norm={err:.2e} max={max_rel(y, exact['out']):.2e}", flush=True)
    assert all(t.dtype == torch.bfloat16 for t in ours.values())
    assert err < 2e-2, err
    for name, e in direct.items():
        assert e <= (OUT_TOL if name.endswith("/out") else GRAD_TOL), (name, direct)


def test_bf16_layer_head_dim_128_with_128_features_close_to_oracle():
    """The fused bf16 prologue at head_dim 128, feature_dim 128 in a whole
    bf16 layer (F = 256, D = 128: the GLA on two D tiles, its k side read
    per kv head), forward and backward."""
    import types
    cfg = types.SimpleNamespace(hidden_size=256, num_attention_heads=2, num_key_value_heads=1)
    torch.manual_seed(1)
    layer = hip_layer.LizardAttention(cfg, 0, window=16, feature_dim=128)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            p.normal_(0, 0.05 if n.split(".")[0] in ("q_proj", "k_proj", "v_proj", "o_proj")
                      else 0.3)
    layer = layer.to(torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 90, 256, generator=g).bfloat16()
    grad = torch.randn(2, 90, 256, generator=g).bfloat16()
    cos, sin = (t.bfloat16()[None].expand(2, 90, 128) for t in lo.rope_cos_sin(90, 128))
    assert layer._fused(*(torch.empty(2, 90, n, dtype=torch.bfloat16) for n in (256, 128, 128)),
                        cos, sin)
    _bf16_layer_case(layer, x, grad, cos, sin, 2, 1, 16, "bf16 layer hd=128 f=128")


def test_config5_bf16_layer_at_size_matches_oracle_layer():
    """One LizardAttention at BASELINE config 5's shape in its own dtype:
    bf16 parameters, input and RoPE tables (theta 500000), hidden 2048, 32
    query / 8 kv heads, head_dim 64, feature_dim 128 (F = 256), window 64, 4
    sinks, on a B=1 slice of its L=4096 sequences: the bf16 MFMA prologue,
    the eight-wave GLA walk and the SWA kernels that bench.py times, forward
    and backward, against the long-L oracle layer in fp64."""
    import types
    cfg = types.SimpleNamespace(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8)
    torch.manual_seed(0)
    layer = hip_layer.LizardAttention(cfg, 0, window=64, num_meta=4, feature_dim=128)
    with torch.no_grad():
        layer.phi_q.weight.normal_(0, 0.3)
        layer.phi_k.weight.normal_(0, 0.3)
        layer.W_gamma.weight.normal_(0, 0.05)   # gates from ~0.1 to ~0.99
        layer.meta_tokens.normal_(0, 1)
        layer.alpha_blend.fill_(0.8)
    layer = layer.bfloat16()
    batch, length = 1, 4096
    g = torch.Generator().manual_seed(5)
    x = torch.randn(batch, length, 2048, generator=g).bfloat16()
    grad = torch.randn(batch, length, 2048, generator=g).bfloat16()
    cos, sin = (t[None].expand(batch, length, 64).bfloat16() for t in lo.rope_cos_sin(length, 64))
    _bf16_layer_case(layer, x, grad, cos, sin, 32, 8, 64, "config5 bf16 layer B=1 L=4096")
