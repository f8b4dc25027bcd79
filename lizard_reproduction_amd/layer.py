"""``LizardAttention`` on the HIP kernels: the drop-in for the reference's
layer with a ``hip`` backend (``src/lizard_attention.py:47-107``).

Same constructor, parameter names, shapes and initialisation, same
``forward(hidden_states, position_embeddings) -> (out, None)`` and the same
``from_llama``, so a checkpoint or a ``LlamaForCausalLM`` whose attention
blocks were swapped for the reference's layer loads into this one unchanged.
The two attention branches run on ``kernels.gla`` and ``kernels.swa``
(hand-written gfx950 kernels); the projections are torch GEMMs.

The layer computes, per token (``src/lizard_attention.py:78-97``):

    q, k, v = split(q_proj(x)), split(k_proj(x)), split(v_proj(x))   # GQA expand
    z       = W_gamma(x)                                             # one gate logit
    fq, fk  = hedgehog(q, phi_q), hedgehog(k, phi_k)                 # F = 2 feature_dim
    qr, kr  = rope(q), rope(k)
    y       = gla(fq, fk, v, logsigmoid(z)) + alpha * swa(qr, kr, v, meta, window)
    out     = o_proj(y)

with everything after the projections in promote(x.dtype, fp32), as the
reference does.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels

BACKENDS = ("hip",)


def hedgehog(x, weight):
    """[softmax(x W^T), softmax(-x W^T)] over the features
    (``src/lizard_attention.py:9-11``)."""
    proj = torch.matmul(x, weight.transpose(0, 1))
    return torch.cat([proj.softmax(-1), (-proj).softmax(-1)], dim=-1)


def rotate(x, cos, sin):
    """rotate_half RoPE with tables [B, L, d] broadcast over the heads (what
    ``transformers``' ``apply_rotary_pos_emb`` does with unsqueeze_dim=1)."""
    half = x.shape[-1] // 2
    rotated = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos.unsqueeze(1) + rotated * sin.unsqueeze(1)


class LizardAttention(nn.Module):
    """Hybrid GLA + sliding-window attention layer
    (``src/lizard_attention.py:47-97``).

    ``config`` needs ``hidden_size``, ``num_attention_heads`` and
    ``num_key_value_heads`` (a ``transformers.LlamaConfig`` has them).  The
    reference's backends are ``"torch"`` (dense L x L math) and ``"triton"``;
    this class is the ``"hip"`` one and accepts only that name.
    """

    def __init__(self, config, layer_idx, window=128, num_meta=4, feature_dim=128,
                 backend="hip"):
        super().__init__()
        if backend not in BACKENDS:
            raise ValueError(f"LizardAttention: backend must be one of {BACKENDS}, got "
                             f"{backend!r} (the dense 'torch' and the 'triton' backends "
                             "are the reference's)")
        self.backend = backend
        hidden = config.hidden_size
        self.layer_idx = layer_idx
        self.heads = config.num_attention_heads
        self.kv_heads = config.num_key_value_heads
        if hidden % self.heads or self.heads % self.kv_heads:
            raise ValueError("LizardAttention: hidden_size must split into heads and "
                             "num_attention_heads into num_key_value_heads groups")
        self.head_dim = hidden // self.heads
        self.window = window
        kv_dim = self.kv_heads * self.head_dim
        self.q_proj = nn.Linear(hidden, hidden, bias=False)
        self.k_proj = nn.Linear(hidden, kv_dim, bias=False)
        self.v_proj = nn.Linear(hidden, kv_dim, bias=False)
        self.o_proj = nn.Linear(hidden, hidden, bias=False)
        self.phi_q = nn.Linear(self.head_dim, feature_dim, bias=False)
        self.phi_k = nn.Linear(self.head_dim, feature_dim, bias=False)
        self.W_gamma = nn.Linear(hidden, 1, bias=False)
        self.meta_tokens = nn.Parameter(torch.zeros(num_meta))
        self.alpha_blend = nn.Parameter(torch.ones(()))
        nn.init.normal_(self.phi_q.weight, std=0.02)
        nn.init.normal_(self.phi_k.weight, std=0.02)
        nn.init.zeros_(self.W_gamma.weight)

    def split(self, x, heads):
        """[B, L, heads * head_dim] -> [B, self.heads, L, head_dim], each kv
        head repeated for its group of query heads."""
        b, n, _ = x.shape
        x = x.view(b, n, heads, self.head_dim).transpose(1, 2)
        return x.repeat_interleave(self.heads // heads, dim=1)

    def forward(self, hidden_states, position_embeddings, **kwargs):
        x = hidden_states
        dtype = torch.promote_types(x.dtype, torch.float32)
        q = self.split(self.q_proj(x), self.heads).to(dtype)
        k = self.split(self.k_proj(x), self.kv_heads).to(dtype)
        v = self.split(self.v_proj(x), self.kv_heads).to(dtype)
        z = self.W_gamma(x).to(dtype).squeeze(-1)
        fq = hedgehog(q, self.phi_q.weight.to(dtype))
        fk = hedgehog(k, self.phi_k.weight.to(dtype))
        cos, sin = (t.to(dtype) for t in position_embeddings)
        qr, kr = rotate(q, cos, sin), rotate(k, cos, sin)
        alpha, meta = self.alpha_blend.to(dtype), self.meta_tokens.to(dtype)
        y = kernels.gla(fq, fk, v, F.logsigmoid(z)).to(dtype)
        y = y + alpha * kernels.swa(qr, kr, v, meta, self.window).to(dtype)
        return self.o_proj(y.to(x.dtype).transpose(1, 2).flatten(2)), None


def from_llama(attention, config, **options):
    """A LizardAttention with a Llama attention block's q/k/v/o projection
    weights, on its device and in its dtype (``src/lizard_attention.py:100-107``)."""
    weight = attention.q_proj.weight
    layer = LizardAttention(config, attention.layer_idx, **options)
    layer = layer.to(weight.device, weight.dtype)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        getattr(layer, name).load_state_dict(getattr(attention, name).state_dict())
    return layer


def to_lizard(model, **options):
    """Swap the self-attention of every decoder layer of a Llama-style model
    (``model.model.layers[i].self_attn``) for a LizardAttention built by
    ``from_llama`` with ``options`` (window, num_meta, feature_dim); returns
    the model (``src/train.py:35-39``)."""
    config = model.config
    for block in model.model.layers:
        block.self_attn = from_llama(block.self_attn, config, **options)
    return model
