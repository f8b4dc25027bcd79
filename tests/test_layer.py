"""CPU checks of the layer: the oracle's dense layer is pinned by its loop
composition and by transformers' LlamaAttention in the softmax limit (the
reference's tests/test_lizard.py:224-288), and the HIP layer's module
surface mirrors the reference's (parameters, init, from_llama, backend
names) without running any kernel."""
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM
from transformers.models.llama.modeling_llama import LlamaAttention, LlamaRotaryEmbedding

from lizard_reproduction_amd import layer as hip_layer
from oracle import lizard_oracle as lo

EXACT = 1e-10


def rel_err(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm()).item()


def tiny_config(layers=1):
    """The reference's tiny Llama (tests/test_lizard.py:94-98)."""
    return LlamaConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, vocab_size=100,
                       attn_implementation="eager")


def tiny_rope(length, start=0, batch=1, dtype=torch.float64):
    x = torch.zeros(1, length, 1, dtype=dtype)
    positions = torch.arange(start, start + length)[None].expand(batch, length)
    return LlamaRotaryEmbedding(tiny_config())(x, positions)


def random_params(seed=0, dtype=torch.float64, window=16, feature_dim=8):
    """Parameters of a layer built like the reference's random_layer
    (tests/test_lizard.py:107-113): every parameter ~ N(0, 0.3)."""
    torch.manual_seed(seed)
    layer = hip_layer.LizardAttention(tiny_config(), 0, window=window, feature_dim=feature_dim)
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.3)
    return {n: p.detach().to(dtype) for n, p in layer.named_parameters()}


def dense(params, x, rope, window=16):
    return lo.lizard_layer(params, x, rope[0], rope[1], 4, 2, window)


def test_oracle_layer_matches_formula_loops():
    params, rope = random_params(), tiny_rope(20)
    x = torch.randn(2, 20, 128).double()
    loop = lo.lizard_layer_loop(params, x, rope[0][0], rope[1][0], 4, 2, 16)
    assert rel_err(dense(params, x, rope), loop) < EXACT


def test_oracle_layer_window_rope_is_relative():
    params = random_params()
    x = torch.randn(2, 20, 128).double()
    shifted = dense(params, x, tiny_rope(20, start=7))
    assert rel_err(shifted, dense(params, x, tiny_rope(20))) < 1e-5


def test_oracle_layer_is_causal_and_batch_independent():
    params, rope = random_params(), tiny_rope(30)
    x = torch.randn(3, 30, 128).double().requires_grad_()
    y = dense(params, x, rope)
    single = torch.cat([dense(params, x[i:i + 1], rope) for i in range(3)])
    assert rel_err(y, single) < EXACT
    y[:, 9].sum().backward()
    assert (x.grad[:, 10:] == 0).all()


def test_oracle_layer_in_the_softmax_limit_is_llama_attention(monkeypatch):
    """GLA branch zeroed, sinks at -1e4, unbounded window: the layer is
    Llama's eager causal attention (tests/test_lizard.py:270-288)."""
    config = tiny_config()
    torch.manual_seed(0)
    llama = LlamaAttention(config, 0).double()
    params = random_params()
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        params[f"{name}.weight"] = getattr(llama, name).weight.detach()
    params["meta_tokens"] = torch.full((4,), -1e4, dtype=torch.float64)
    params["alpha_blend"] = torch.ones((), dtype=torch.float64)
    monkeypatch.setattr(lo, "gla", lambda fq, fk, v, g: torch.zeros_like(v))
    x, rope = torch.randn(2, 30, 128).double(), tiny_rope(30, batch=2)
    mask = torch.full((30, 30), float("-inf")).triu(1).double()[None, None]
    expected, _ = llama(hidden_states=x, position_embeddings=rope, attention_mask=mask)
    assert rel_err(dense(params, x, rope, window=10**6), expected) < 1e-6


def test_oracle_layer_catches_a_wrong_kv_head_map():
    """A planted mistake (kv heads tiled instead of repeated per group)
    fails the loop check, so that check pins the GQA expansion."""
    params, rope = random_params(), tiny_rope(12)
    x = torch.randn(1, 12, 128).double()
    loop = lo.lizard_layer_loop(params, x, rope[0][0], rope[1][0], 4, 2, 16)
    good = torch.Tensor.repeat_interleave

    def tiled(t, n, dim):
        return t.repeat(*[n if d == dim else 1 for d in range(t.dim())])
    try:
        torch.Tensor.repeat_interleave = lambda t, n, dim: tiled(t, n, dim)
        wrong = dense(params, x, rope)
    finally:
        torch.Tensor.repeat_interleave = good
    assert rel_err(wrong, loop) > 1e-3
    assert rel_err(dense(params, x, rope), loop) < EXACT


# -- the HIP layer's module surface (no kernel runs here) ---------------------

def reference_shapes(config, window, num_meta, feature_dim):
    """Parameter names and shapes of src/lizard_attention.py:49-71."""
    hidden, heads, kv = config.hidden_size, config.num_attention_heads, config.num_key_value_heads
    hd = hidden // heads
    return {"q_proj.weight": (hidden, hidden), "k_proj.weight": (kv * hd, hidden),
            "v_proj.weight": (kv * hd, hidden), "o_proj.weight": (hidden, hidden),
            "phi_q.weight": (feature_dim, hd), "phi_k.weight": (feature_dim, hd),
            "W_gamma.weight": (1, hidden), "meta_tokens": (num_meta,), "alpha_blend": ()}


def test_layer_parameters_and_init_mirror_the_reference():
    layer = hip_layer.LizardAttention(tiny_config(), 3, window=16, num_meta=5, feature_dim=8)
    shapes = {n: tuple(p.shape) for n, p in layer.named_parameters()}
    assert shapes == reference_shapes(tiny_config(), 16, 5, 8)
    assert (layer.W_gamma.weight == 0).all() and (layer.meta_tokens == 0).all()
    assert layer.alpha_blend.item() == 1.0
    assert 0.005 < layer.phi_q.weight.std().item() < 0.05
    assert (layer.layer_idx, layer.window, layer.heads, layer.kv_heads, layer.head_dim) == \
        (3, 16, 4, 2, 32)


@pytest.mark.parametrize("backend", ["torch", "triton", "cuda"])
def test_layer_rejects_other_backends(backend):
    with pytest.raises(ValueError, match="backend"):
        hip_layer.LizardAttention(tiny_config(), 0, backend=backend)


def test_from_llama_copies_projections_and_keeps_dtype():
    config = tiny_config()
    llama = LlamaAttention(config, 0).to(torch.bfloat16)
    layer = hip_layer.from_llama(llama, config, window=16, feature_dim=8)
    assert all(p.dtype == torch.bfloat16 for p in layer.parameters())
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        assert torch.equal(getattr(layer, name).weight, getattr(llama, name).weight)


def test_to_lizard_swaps_every_block():
    model = LlamaForCausalLM(tiny_config(layers=2))
    hip_layer.to_lizard(model, window=16, num_meta=4, feature_dim=8, backend="hip")
    assert all(isinstance(b.self_attn, hip_layer.LizardAttention) for b in model.model.layers)
    assert [b.self_attn.layer_idx for b in model.model.layers] == [0, 1]


@pytest.mark.parametrize("prompt, window", [(5, 8), (8, 8), (21, 8), (3, 1)])
def test_cache_ring_holds_the_last_window_positions(prompt, window):
    """LizardCache.put (plain torch, no kernels): after a prompt of any
    length and then single-token writes, slot p % window holds position p for
    the last `window` positions -- what the SWA decode kernel reads."""
    b, kv, hd = 2, 3, 4
    k = torch.zeros(b, kv, window, hd, dtype=torch.bfloat16)
    cache = hip_layer.LizardCache(None, k, torch.zeros_like(k), 0)

    def rows(p0, n):   # position p's key is filled with the value p, its value with -p
        pos = torch.arange(p0, p0 + n, dtype=torch.float32).view(1, 1, n, 1)
        return pos.expand(b, kv, n, hd).bfloat16(), (-pos).expand(b, kv, n, hd).bfloat16()
    cache.put(*rows(0, prompt), 0)
    end = prompt
    for p in range(prompt, prompt + 5):
        cache.put(*rows(p, 1), p)
        end = p + 1
        for q in range(max(0, end - window), end):
            assert torch.all(cache.k[:, :, q % window] == q), (p, q)
            assert torch.all(cache.v[:, :, q % window] == -q), (p, q)


# -- the long-L oracle layer (banded SWA, chunked GLA) -----------------------

@pytest.mark.parametrize("length, window, block", [(1, 4, 64), (77, 16, 16), (150, 64, 64),
                                                   (130, 1, 64), (97, 200, 16), (64, 64, 64)])
def test_banded_swa_equals_dense_awa(length, window, block):
    g = torch.Generator().manual_seed(length)
    q, k, v = (torch.randn(2, 3, length, 20, generator=g, dtype=torch.float64)
               .requires_grad_() for _ in range(3))
    meta = torch.randn(4, generator=g, dtype=torch.float64).requires_grad_()
    dy = torch.randn(2, 3, length, 20, generator=g, dtype=torch.float64)
    dense_y = lo.awa(q, k, v, meta, window)
    dense_y.backward(dy)
    grads = [t.grad.clone() for t in (q, k, v, meta)]
    for t in (q, k, v, meta):
        t.grad = None
    band = lo.awa_banded(q, k, v, meta, window, block=block)
    band.backward(dy)
    assert rel_err(band, dense_y) < EXACT
    for t, ref in zip((q, k, v, meta), grads):
        assert rel_err(t.grad, ref) < EXACT


def test_banded_swa_without_sinks_equals_dense_awa():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 2, 90, 16, generator=g, dtype=torch.float64) for _ in range(3))
    meta = torch.empty(0, dtype=torch.float64)
    assert rel_err(lo.awa_banded(q, k, v, meta, 32), lo.awa(q, k, v, meta, 32)) < EXACT


@pytest.mark.parametrize("length, window", [(40, 16), (130, 16), (200, 100), (256, 64)])
def test_banded_oracle_layer_equals_dense_layer(length, window):
    """The long-L oracle layer (chunked GLA, banded SWA) against the dense
    one in fp64: output, input gradient and every parameter gradient."""
    params = random_params(window=window)
    for p in params.values():
        p.requires_grad_()
    rope = tiny_rope(length, batch=2)
    g = torch.Generator().manual_seed(length)
    x = torch.randn(2, length, 128, generator=g, dtype=torch.float64).requires_grad_()
    dy = torch.randn(2, length, 128, generator=g, dtype=torch.float64)
    ref = lo.lizard_layer(params, x, rope[0], rope[1], 4, 2, window)
    ref.backward(dy)
    ref_grads = {n: p.grad.clone() for n, p in params.items()}
    ref_dx = x.grad.clone()
    for p in list(params.values()) + [x]:
        p.grad = None
    band = lo.lizard_layer_banded(params, x, rope[0], rope[1], 4, 2, window)
    band.backward(dy)
    assert rel_err(band, ref) < EXACT
    assert rel_err(x.grad, ref_dx) < EXACT
    for n, p in params.items():
        assert rel_err(p.grad, ref_grads[n]) < EXACT, n


def test_banded_oracle_layer_catches_a_window_off_by_one(monkeypatch):
    """A planted mistake in the banded window (one key too many) fails the
    check against the dense layer."""
    params, rope = random_params(), tiny_rope(70)
    x = torch.randn(1, 70, 128, dtype=torch.float64)
    good = lo.awa_banded
    monkeypatch.setattr(lo, "awa_banded", lambda q, k, v, m, w, block=64: good(q, k, v, m, w + 1,
                                                                                block))
    wrong = lo.lizard_layer_banded(params, x, rope[0], rope[1], 4, 2, 16)
    assert rel_err(wrong, lo.lizard_layer(params, x, rope[0], rope[1], 4, 2, 16)) > 1e-4


def test_layer_takes_any_even_head_dim_up_to_the_swa_limit():
    """The reference's layer takes any head_dim / feature_dim
    (src/lizard_attention.py:47-66); the fused prologue covers head_dim 32,
    64, 128 (feature_dim up to 128, bf16 at 128 x 128), the rest runs its
    torch ops before the same kernels.  The SWA kernels bound head_dim."""
    import types

    def cfg(hidden, heads):
        return types.SimpleNamespace(hidden_size=hidden, num_attention_heads=heads,
                                     num_key_value_heads=1)
    for hidden, heads, f in ((256, 2, 128), (192, 2, 24), (512, 2, 256)):
        layer = hip_layer.LizardAttention(cfg(hidden, heads), 0, feature_dim=f)
        assert layer.head_dim == hidden // heads
    with pytest.raises(ValueError, match="head_dim"):
        hip_layer.LizardAttention(cfg(1024, 2), 0)            # head_dim 512 > 256
    with pytest.raises(ValueError, match="head_dim"):
        hip_layer.LizardAttention(cfg(99, 3), 0)              # odd head_dim
    assert hip_layer.prologue_supported(128, 128, bf16=True)
    assert not hip_layer.prologue_supported(128, 128, bf16=False)
    assert hip_layer.prologue_supported(128, 64, bf16=False)
    assert not hip_layer.prologue_supported(96, 16)


def _sweep_layer(seed=0, heads=4, kv=2, hd=24, f=12, sinks=3, window=5):
    import types
    cfg = types.SimpleNamespace(hidden_size=heads * hd, num_attention_heads=heads,
                                num_key_value_heads=kv)
    torch.manual_seed(seed)
    layer = hip_layer.LizardAttention(cfg, 0, window=window, num_meta=sinks, feature_dim=f)
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.3)
    return {n: p.detach().double() for n, p in layer.named_parameters()}


def _layer_grads(fn, params, x, grad):
    params = {n: p.detach().clone().requires_grad_() for n, p in params.items()}
    xd = x.detach().clone().requires_grad_()
    y = fn(params, xd)
    y.backward(grad)
    out = {n: p.grad for n, p in params.items()}
    out["dx"], out["out"] = xd.grad, y.detach()
    return out


@pytest.mark.parametrize("bf16_layer", [False, True])
@pytest.mark.parametrize("length, window", [(30, 5), (130, 100)])
def test_rounded_oracle_layer_without_rounding_is_the_oracle_layer(bf16_layer, length, window):
    """lo.lizard_layer_rounded with its rounding off is the dense oracle
    layer: output, input gradient and every parameter gradient in fp64 (L =
    130 spans three 64-token GLA chunks and, at window 5, several SWA
    blocks), in both of its layer modes."""
    params = _sweep_layer(window=window)
    g = torch.Generator().manual_seed(length)
    x = torch.randn(2, length, 96, generator=g, dtype=torch.float64)
    grad = torch.randn(2, length, 96, generator=g, dtype=torch.float64)
    cos, sin = (t[None].expand(2, length, 24) for t in lo.rope_cos_sin(length, 24))
    dense_g = _layer_grads(lambda p, xd: lo.lizard_layer(p, xd, cos, sin, 4, 2, window),
                           params, x, grad)
    plain = _layer_grads(lambda p, xd: lo.lizard_layer_rounded(
        p, xd, cos, sin, 4, 2, window, rounded=False, bf16_layer=bf16_layer), params, x, grad)
    for name in dense_g:
        assert rel_err(plain[name], dense_g[name]) < EXACT, name


def test_rounded_oracle_layer_applies_its_rounding_points():
    """With rounding on, every output and gradient moves off the exact layer
    (the rounding is really applied), by bf16-sized amounts except the sink
    gradient: there the sink probabilities exp(meta - lse_i) of this draw's
    large scores (|q.k|/sqrt(d) ~ 40) move with the absolute error that the
    bf16 q and k put into the scores, so that gradient is the rounding's own
    (the HIP kernels take the same bf16 q and k, and are compared with this
    model rather than with the exact layer for that reason).  The bf16-layer
    mode adds its own rounding points (projections, blended y, output); the
    SWA branch's P rounding moves its output; and round_bf16 is the bf16
    cast both ways."""
    params = _sweep_layer()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 70, 96, generator=g, dtype=torch.float64)
    grad = torch.randn(2, 70, 96, generator=g, dtype=torch.float64)
    cos, sin = (t[None].expand(2, 70, 24) for t in lo.rope_cos_sin(70, 24))
    runs = {mode: _layer_grads(lambda p, xd: lo.lizard_layer_rounded(
        p, xd, cos, sin, 4, 2, 5, rounded=mode != "exact", bf16_layer=mode == "bf16"),
        params, x, grad) for mode in ("exact", "fp32", "bf16")}
    for name in runs["exact"]:
        d32 = rel_err(runs["fp32"][name], runs["exact"][name])
        d16 = rel_err(runs["bf16"][name], runs["fp32"][name])
        assert d32 > 1e-6 and (d32 < 2e-2 or name == "meta_tokens"), (name, d32)
        assert d16 > 1e-6, (name, d16)
    q, k, v = (torch.randn(1, 2, 90, 16, generator=g, dtype=torch.float64) for _ in range(3))
    meta = torch.randn(3, generator=g, dtype=torch.float64)
    exact, rnd = (lo.awa_banded(q, k, v, meta, 20, round_p=r) for r in (False, True))
    assert 1e-6 < rel_err(rnd, exact) < 1e-2
    t = torch.randn(1000, generator=g, dtype=torch.float64).requires_grad_()
    up = torch.randn(1000, generator=g, dtype=torch.float64)
    lo.round_bf16(t).backward(up)
    assert torch.equal(lo.round_bf16(t).detach(), t.detach().bfloat16().double())
    assert torch.equal(t.grad, up.bfloat16().double())
