"""``LizardAttention`` on the HIP kernels: the drop-in for the reference's
layer with a ``hip`` backend (``src/lizard_attention.py:47-107``).

Same constructor, parameter names, shapes and initialisation, same
``forward(hidden_states, position_embeddings) -> (out, None)`` and the same
``from_llama``, so a checkpoint or a ``LlamaForCausalLM`` whose attention
blocks were swapped for the reference's layer loads into this one unchanged.

The layer computes, per token (``src/lizard_attention.py:78-97``):

    q, k, v = split(q_proj(x)), split(k_proj(x)), split(v_proj(x))   # GQA expand
    z       = W_gamma(x)                                             # one gate logit
    fq, fk  = hedgehog(q, phi_q), hedgehog(k, phi_k)                 # F = 2 feature_dim
    qr, kr  = rope(q), rope(k)
    y       = gla(fq, fk, v, logsigmoid(z)) + alpha * swa(qr, kr, v, meta, window)
    out     = o_proj(y)

with everything after the projections in promote(x.dtype, fp32).  The
projections and the gate logit are torch GEMMs; everything from the
projection outputs to o_proj's input runs on HIP kernels: the fused
prologue (GQA expand, Hedgehog feature maps, RoPE and the bf16 casts, one
pass over q/k/v), the GLA kernels (which take the logit z and form
logsigmoid(z) and its derivative themselves) and the SWA kernels, and the
fused blend + transpose, one autograd node for all of them (``_Core``).

Decoding (no counterpart in the reference, which has no decode path):
``prefill`` runs the forward over a prompt and returns a ``LizardCache`` --
the GLA recurrent state after the prompt and a ring buffer of the last
``window`` keys (RoPE applied) and values per kv head -- and ``step`` runs
one token per sequence from it, each output equal (up to rounding) to the
forward's row for that position.
"""
import functools

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, kernels

BACKENDS = ("hip",)
MAX_HEAD_DIM = 256       # lz_swa_*: dim <= 256
MAX_FEATURE_DIM = 2048   # lz_gla_*: F = 2 feature_dim <= LZ_GLA_MAX_DIM


def _stream(t):
    return torch._C._cuda_getCurrentRawStream(t.device.index)


@functools.lru_cache(maxsize=64)
def _prologue_ws(b, length, heads, kv, hd, f):
    return _lib.load().lz_layer_prologue_bwd_workspace_bytes(b, length, heads, kv, hd, f)


def prologue_supported(head_dim, feature_dim, bf16=True):
    """Shapes the fused prologue takes: head_dim 32, 64 or 128; feature_dim a
    multiple of 4 up to 128, up to 64 with head_dim 128 when its arithmetic
    is fp32 (bf16 inputs take 128 there too).  Other shapes take the
    reference's torch ops before the same GLA and SWA kernels."""
    return (head_dim in (32, 64, 128) and feature_dim > 0 and feature_dim % 4 == 0
            and feature_dim <= (64 if head_dim == 128 and not bf16 else 128))


def _all_bf16(*tensors):
    """The prologue's arithmetic is bf16 only when every input is bf16 (else
    they are all widened to fp32, exactly, as the reference promotes them)."""
    return all(t.dtype == torch.bfloat16 for t in tensors)


def _tables(cos, sin, batch, length, head_dim, dtype):
    """RoPE tables as contiguous [B, L, hd] or [L, hd] of ``dtype``; returns
    (cos, sin, batched)."""
    if cos.shape != sin.shape:
        raise ValueError(f"LizardAttention: cos and sin shapes differ: {tuple(cos.shape)} "
                         f"vs {tuple(sin.shape)}")
    if cos.dim() == 3 and cos.shape[0] == 1:
        cos, sin = cos[0], sin[0]
    if cos.dim() == 2:
        ok, batched = tuple(cos.shape) == (length, head_dim), 0
    else:
        ok, batched = tuple(cos.shape) == (batch, length, head_dim), 1
    if not ok:
        raise ValueError(f"LizardAttention: position embeddings of shape {tuple(cos.shape)} "
                         f"do not match B={batch}, L={length}, head_dim={head_dim}")
    return cos.to(dtype).contiguous(), sin.to(dtype).contiguous(), batched


def prologue_forward(qp, kp, vp, wq, wk, cos, sin, heads, kv_heads, with_fq=True):
    """One ``lz_layer_prologue_fwd`` launch: the q/k/v projection outputs
    ([B, L, heads * hd], [B, L, kv_heads * hd]) and phi weights ([f, hd]) to
    the bf16 kernel operands fq ([B, heads, L, 2f]), qr ([B, heads, L, hd]),
    fk ([B, kv_heads, L, 2f]) and kr, v ([B, kv_heads, L, hd]): the key side
    stays per kv head, and the GLA and SWA kernels read each query head's
    from its kv head (the reference's repeat_interleave, not materialised).
    Returns those five and the tuple ``prologue_backward`` needs; without
    ``with_fq`` fq is None and not computed (``kernels.gla_forward_phi``
    forms it inside the GLA walk)."""
    if qp.dim() != 3 or heads <= 0 or kv_heads <= 0 or heads % kv_heads or \
            qp.shape[-1] % heads:
        raise ValueError(f"prologue_forward: q must be [B, L, heads * head_dim] with kv_heads "
                         f"dividing heads; got {tuple(qp.shape)}, heads={heads}, "
                         f"kv_heads={kv_heads}")
    b, length, _ = qp.shape
    hd = qp.shape[-1] // heads
    f = wq.shape[0]
    for name, t, shape in (("k", kp, (b, length, kv_heads * hd)),
                           ("v", vp, (b, length, kv_heads * hd)),
                           ("wq", wq, (f, hd)), ("wk", wk, (f, hd))):
        if tuple(t.shape) != shape:
            raise ValueError(f"prologue_forward: {name} must be {shape}, got {tuple(t.shape)}")
    dtype = torch.bfloat16 if _all_bf16(qp, kp, vp, wq, wk, cos, sin) else torch.float32
    qp, kp, vp, wq, wk = (t.to(dtype).contiguous() for t in (qp, kp, vp, wq, wk))
    cos, sin, batched = _tables(cos, sin, b, length, hd, dtype)
    dev = qp.device
    fq = torch.empty(b, heads, length, 2 * f, device=dev, dtype=torch.bfloat16) if with_fq \
        else None
    fk = torch.empty(b, kv_heads, length, 2 * f, device=dev, dtype=torch.bfloat16)
    qr = torch.empty(b, heads, length, hd, device=dev, dtype=torch.bfloat16)
    kr = torch.empty(b, kv_heads, length, hd, device=dev, dtype=torch.bfloat16)
    v = torch.empty_like(kr)
    rc = _lib.load().lz_layer_prologue_fwd(
        qp.data_ptr(), kp.data_ptr(), vp.data_ptr(), wq.data_ptr(), wk.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), batched, fq.data_ptr() if with_fq else None,
        fk.data_ptr(), qr.data_ptr(),
        kr.data_ptr(), v.data_ptr(), int(dtype == torch.bfloat16), b, length, heads, kv_heads,
        hd, f, _stream(qp))
    _lib.check(rc, "lz_layer_prologue_fwd")
    saved = (qp, kp, wq, wk, cos, sin, (b, length, heads, kv_heads, hd, f, batched))
    return fq, fk, qr, kr, v, saved


def prologue_backward(saved, dfq, dfk, dqr, dkr, dv, dv2=None):
    """One ``lz_layer_prologue_bwd`` launch from the gradients of fq, fk, qr,
    kr and v (taken as bf16; dv2: an optional second gradient of v, added in
    fp32); returns dq, dk, dv of the projection outputs (in the arithmetic
    dtype) and dWq, dWk (fp32)."""
    qp, kp, wq, wk, cos, sin, (b, length, heads, kv, hd, f, batched) = saved
    # every gradient is per query head (the kernels' gradients of the k-side
    # operands are each query head's share; the kernel sums them per group)
    for name, g, n in (("dfq", dfq, 2 * f), ("dfk", dfk, 2 * f), ("dqr", dqr, hd),
                       ("dkr", dkr, hd), ("dv", dv, hd), ("dv2", dv2, hd)):
        if g is not None and tuple(g.shape) != (b, heads, length, n):
            raise ValueError(f"prologue_backward: {name} must be {(b, heads, length, n)}, got "
                             f"{tuple(g.shape)}")
    grads = [None if g is None else g.to(torch.bfloat16).contiguous()
             for g in (dfq, dfk, dqr, dkr, dv, dv2)]
    dq, dk, dvp = torch.empty_like(qp), torch.empty_like(kp), torch.empty_like(kp)
    dwq = torch.empty(wq.shape, device=wq.device, dtype=torch.float32)
    dwk = torch.empty_like(dwq)
    nbytes = _prologue_ws(b, length, heads, kv, hd, f)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=qp.device)
    rc = _lib.load().lz_layer_prologue_bwd(
        qp.data_ptr(), kp.data_ptr(), wq.data_ptr(), wk.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), batched, *(None if g is None else g.data_ptr() for g in grads),
        dq.data_ptr(), dk.data_ptr(), dvp.data_ptr(), dwq.data_ptr(), dwk.data_ptr(),
        int(qp.dtype == torch.bfloat16), b, length, heads, kv, hd, f, ws.data_ptr(), nbytes,
        _stream(qp))
    _lib.check(rc, "lz_layer_prologue_bwd")
    return dq, dk, dvp, dwq, dwk


def combine_forward(yg, ys, alpha, out_dtype):
    """``lz_layer_combine_fwd``: y_gla + alpha * y_swa ([B, H, L, hd] bf16;
    alpha fp32 [1]) as [B, L, H * hd] in out_dtype (bf16 or fp32)."""
    b, heads, length, hd = yg.shape
    out = torch.empty(b, length, heads * hd, device=yg.device, dtype=out_dtype)
    rc = _lib.load().lz_layer_combine_fwd(yg.data_ptr(), ys.data_ptr(), alpha.data_ptr(),
                                          out.data_ptr(), int(out_dtype == torch.bfloat16), b,
                                          heads, length, hd, _stream(yg))
    _lib.check(rc, "lz_layer_combine_fwd")
    return out


def combine_backward(dout, ys, alpha):
    """``lz_layer_combine_bwd``: bf16 gradients of y_gla and y_swa and the
    fp32 gradient of alpha ([1])."""
    b, heads, length, hd = ys.shape
    dyg, dys = torch.empty_like(ys), torch.empty_like(ys)
    dalpha = torch.empty(1, device=ys.device, dtype=torch.float32)
    lib = _lib.load()
    nbytes = lib.lz_layer_combine_bwd_workspace_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=ys.device)
    rc = lib.lz_layer_combine_bwd(dout.data_ptr(), ys.data_ptr(), alpha.data_ptr(),
                                  dyg.data_ptr(), dys.data_ptr(), dalpha.data_ptr(),
                                  int(dout.dtype == torch.bfloat16), b, heads, length, hd,
                                  ws.data_ptr(), nbytes, _stream(ys))
    _lib.check(rc, "lz_layer_combine_bwd")
    return dyg, dys, dalpha


class _Core(torch.autograd.Function):
    """Everything from the projection outputs to o_proj's input as one
    autograd node (src/lizard_attention.py:73-97): prologue, GLA, SWA and
    the blend, forward and backward.  The kernels hand each other bf16
    gradients of their bf16 operands (the reference's layer keeps fp32 ones
    for its fp32 intermediates): half the bytes on the backward's largest
    streams, for one extra bf16 rounding of each gradient (2^-9 relative,
    the size of the rounding its bf16 projections already take)."""

    @staticmethod
    def forward(ctx, qp, kp, vp, wq, wk, z, meta, alpha, cos, sin, heads, kv_heads,
                window, out_dtype):
        # z is the gate logit [B, L]: the GLA kernels form log_gamma =
        # logsigmoid(z) where they read it and return the gradient of z
        # (src/lizard_attention.py:92, F.logsigmoid, fused)
        fq, fk, qr, kr, v, saved = prologue_forward(qp, kp, vp, wq, wk, cos, sin, heads,
                                                    kv_heads)
        lg = z.float().contiguous()
        meta32 = meta.float().contiguous()
        alpha32 = alpha.detach().float().reshape(1).contiguous()
        grad = any(ctx.needs_input_grad[:8])
        y_gla, state = kernels.gla_forward(fq, fk, v, lg, keep_state=grad, gate_logit=True)
        y_swa, lse = kernels.swa_forward(qr, kr, v, meta32, window)
        odt = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
        out = combine_forward(y_gla, y_swa, alpha32, odt)
        if grad:
            ctx.save_for_backward(fq, fk, qr, kr, v, lg, meta32, lse, y_swa, alpha32,
                                  *saved[:6])
            ctx.state, ctx.sizes = state, saved[6]
        ctx.window = window
        ctx.dtypes = (qp.dtype, kp.dtype, vp.dtype, wq.dtype, wk.dtype, z.dtype,
                      meta.dtype, alpha.dtype)
        return out.to(out_dtype)

    @staticmethod
    def backward(ctx, dout):
        fq, fk, qr, kr, v, lg, meta32, lse, y_swa, alpha32, *saved = ctx.saved_tensors
        saved = tuple(saved) + (ctx.sizes,)
        odt = torch.bfloat16 if dout.dtype == torch.bfloat16 else torch.float32
        dyg, dys, dalpha = combine_backward(dout.to(odt).contiguous(), y_swa, alpha32)
        bf = torch.bfloat16
        dfq, dfk, dv_gla, dz = kernels.gla_backward(fq, fk, v, lg, dyg, ctx.state, bf,
                                                    gate_logit=True)
        dqr, dkr, dv_swa, dmeta = kernels.swa_backward(qr, kr, v, meta32, lse, dys, ctx.window,
                                                       bf)
        dq, dk, dvp, dwq, dwk = prologue_backward(saved, dfq, dfk, dqr, dkr, dv_gla, dv_swa)
        grads = (dq, dk, dvp, dwq, dwk, dz, dmeta, dalpha.reshape(()))
        return tuple(g.to(d) for g, d in zip(grads, ctx.dtypes)) + (None,) * 6


class LizardCache:
    """Decode state of one layer: ``state`` fp32 [B, heads, F*hd + F] (the
    GLA recurrent state S, z; F = 2 feature_dim), ``k`` and ``v`` bf16
    [B, kv_heads, window, hd] (position p in slot p % window, RoPE applied
    to k), ``pos`` the absolute position of the next token."""

    def __init__(self, state, k, v, pos):
        self.state, self.k, self.v, self.pos = state, k, v, pos

    def put(self, kr, v, p0):
        """Write positions p0 .. p0 + n - 1 of kr, v ([B, kv_heads, n, hd]);
        only the last ``window`` of them stay."""
        window = self.k.shape[2]
        n = kr.shape[2]
        if n == 1:   # a decode step: one slot, plain copies
            self.k[:, :, p0 % window] = kr[:, :, 0]
            self.v[:, :, p0 % window] = v[:, :, 0]
            return
        first = max(0, n - window)
        slots = torch.arange(p0 + first, p0 + n, device=kr.device) % window
        self.k[:, :, slots] = kr[:, :, first:]
        self.v[:, :, slots] = v[:, :, first:]


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
        if not 0 < self.head_dim <= MAX_HEAD_DIM or self.head_dim % 2 or \
                not 0 < feature_dim <= MAX_FEATURE_DIM:
            raise ValueError(f"LizardAttention: head_dim {self.head_dim} / feature_dim "
                             f"{feature_dim} unsupported (an even head_dim up to {MAX_HEAD_DIM}, "
                             f"the SWA kernels' limit; feature_dim up to {MAX_FEATURE_DIM}, "
                             "the GLA kernels' F = 2 feature_dim)")
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

    def _fused(self, qp, kp, vp, cos, sin):
        """Whether the fused prologue takes this layer's shapes and dtypes,
        decided from the tensors ``prologue_forward`` itself reads (the
        projection outputs, both phi weights and the RoPE tables), so that
        the two never disagree on the arithmetic dtype."""
        bf16 = _all_bf16(qp, kp, vp, self.phi_q.weight, self.phi_k.weight, cos, sin)
        return prologue_supported(self.head_dim, self.phi_q.weight.shape[0], bf16)

    def _phi_walk(self, qp, kp, vp, cos, sin):
        """Whether the GLA walk can form fq itself (``kernels.gla_forward_phi``):
        a bf16 layer at head_dim 64 with feature_dim 128 (F = 256)."""
        return (self.head_dim == 64 and self.phi_q.weight.shape[0] == 128 and
                _all_bf16(qp, kp, vp, self.phi_q.weight, self.phi_k.weight, cos, sin))

    def _needs_grad(self, x):
        return torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _inference(self, qp, kp, vp, z, cos, sin, out_dtype, final_state=False):
        """The forward without autograd with fq formed inside the GLA walk:
        the prologue writes fk, qr, kr, v only; ``gla_forward_phi`` reads the
        q projection rows and phi_q instead of fq.  Returns (out before
        o_proj, the GLA state after the last token or None, kr, v)."""
        _, fk, qr, kr, v, _ = prologue_forward(qp, kp, vp, self.phi_q.weight, self.phi_k.weight,
                                               cos, sin, self.heads, self.kv_heads,
                                               with_fq=False)
        y_gla, state = kernels.gla_forward_phi(qp, self.phi_q.weight, fk, v,
                                               z.float().contiguous(), self.heads,
                                               gate_logit=True, final_state=final_state)
        y_swa, _ = kernels.swa_forward(qr, kr, v, self.meta_tokens.detach().float().contiguous(),
                                       self.window)
        alpha = self.alpha_blend.detach().float().reshape(1).contiguous()
        odt = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
        return combine_forward(y_gla, y_swa, alpha, odt).to(out_dtype), state, kr, v

    def forward(self, hidden_states, position_embeddings, **kwargs):
        x = hidden_states
        dtype = torch.promote_types(x.dtype, torch.float32)
        kernels._refuse_capture("LizardAttention")
        if x.device.type != "cuda":
            raise ValueError("LizardAttention (hip backend) needs its input on a ROCm GPU")
        z = self.W_gamma(x).to(dtype).squeeze(-1)
        cos, sin = position_embeddings
        qp, kp, vp = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        if not self._fused(qp, kp, vp, cos, sin):
            y = self._unfused(qp, kp, vp, F.logsigmoid(z), cos, sin, dtype).to(x.dtype)
            return self.o_proj(y.transpose(1, 2).flatten(2)), None
        if not self._needs_grad(x) and self._phi_walk(qp, kp, vp, cos, sin):
            return self.o_proj(self._inference(qp, kp, vp, z, cos, sin, x.dtype)[0]), None
        y = _Core.apply(qp, kp, vp, self.phi_q.weight, self.phi_k.weight, z, self.meta_tokens,
                        self.alpha_blend, cos, sin, self.heads, self.kv_heads, self.window,
                        x.dtype)
        return self.o_proj(y), None

    def _unfused(self, qp, kp, vp, log_gamma, cos, sin, dtype):
        """The layer between the projections and o_proj for shapes the fused
        prologue does not take: the reference's own torch ops -- heads split
        and repeated per group, Hedgehog maps, rotate_half RoPE, promotion to
        ``dtype`` (src/lizard_attention.py:73-88) -- in front of the same HIP
        GLA and SWA operators, blended as y_gla + alpha y_swa (:90-93)."""
        b, n, _ = qp.shape

        def heads_of(t, count):
            t = t.view(b, n, count, self.head_dim).transpose(1, 2)
            return t.repeat_interleave(self.heads // count, dim=1).to(dtype)

        def hedgehog(t, w):
            p = torch.matmul(t, w.to(dtype).transpose(0, 1))
            return torch.cat([p.softmax(-1), (-p).softmax(-1)], dim=-1)

        c, s = (t.to(dtype) for t in (cos, sin))
        c, s = (t.unsqueeze(1) if t.dim() == 3 else t for t in (c, s))
        half = self.head_dim // 2

        def rope(t):
            return t * c + torch.cat([-t[..., half:], t[..., :half]], dim=-1) * s
        q, k, v = heads_of(qp, self.heads), heads_of(kp, self.kv_heads), heads_of(vp, self.kv_heads)
        y_gla = kernels.gla(hedgehog(q, self.phi_q.weight), hedgehog(k, self.phi_k.weight), v,
                            log_gamma).to(dtype)
        y_swa = kernels.swa(rope(q), rope(k), v, self.meta_tokens.to(dtype), self.window)
        return y_gla + self.alpha_blend.to(dtype) * y_swa.to(dtype)

    # -- decoding -----------------------------------------------------------

    def new_cache(self, batch, device=None):
        """The cache of an empty prefix (zeros, pos 0)."""
        device = device if device is not None else self.q_proj.weight.device
        nf = 2 * self.phi_q.weight.shape[0]
        state = kernels.new_state(batch, self.heads, nf, self.head_dim, device)
        shape = (batch, self.kv_heads, self.window, self.head_dim)
        k = torch.zeros(shape, device=device, dtype=torch.bfloat16)
        return LizardCache(state, k, torch.zeros_like(k), 0)

    def _operands(self, x, position_embeddings, projections=None):
        kernels._refuse_capture("LizardAttention")
        if x.device.type != "cuda":
            raise ValueError("LizardAttention (hip backend) needs its input on a ROCm GPU")
        nf = 2 * self.phi_q.weight.shape[0]
        cos, sin = position_embeddings
        qp, kp, vp = projections or (self.q_proj(x), self.k_proj(x), self.v_proj(x))
        if not self._fused(qp, kp, vp, cos, sin) or not kernels.gla_native(nf, self.head_dim):
            raise ValueError(f"LizardAttention.prefill/step: decoding takes the fused prologue's "
                             f"shapes and the GLA decode kernels' (F = {nf}, D = "
                             f"{self.head_dim} is not one: F <= 256, D <= 128, D <= 64 when "
                             "F > 128)")
        # the gate logit: the GLA kernels take logsigmoid of it themselves
        z = self.W_gamma(x).float().squeeze(-1).contiguous()
        fq, fk, qr, kr, v, _ = prologue_forward(qp, kp, vp, self.phi_q.weight,
                                                self.phi_k.weight, cos, sin, self.heads,
                                                self.kv_heads)
        return z, fq, fk, qr, kr, v

    def _out(self, y_gla, y_swa, x):
        alpha = self.alpha_blend.detach().float().reshape(1).contiguous()
        odt = torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float32
        return self.o_proj(combine_forward(y_gla, y_swa, alpha, odt).to(x.dtype))

    @torch.no_grad()
    def prefill(self, hidden_states, position_embeddings):
        """``forward`` over a prompt [B, L, hidden] (no autograd) that also
        returns the decode cache after it: ``(out, cache)``."""
        x = hidden_states
        cache = self.new_cache(x.shape[0], x.device)
        cos, sin = position_embeddings
        qp, kp, vp = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        if self._fused(qp, kp, vp, cos, sin) and self._phi_walk(qp, kp, vp, cos, sin):
            kernels._refuse_capture("LizardAttention")
            z = self.W_gamma(x).float().squeeze(-1)
            y, state, kr, v = self._inference(qp, kp, vp, z, cos, sin, x.dtype, final_state=True)
            out = self.o_proj(y)
        else:
            z, fq, fk, qr, kr, v = self._operands(x, position_embeddings, (qp, kp, vp))
            y_gla, state = kernels.gla_prefill(fq, fk, v, z, gate_logit=True)
            y_swa, _ = kernels.swa_forward(qr, kr, v,
                                           self.meta_tokens.detach().float().contiguous(),
                                           self.window)
            out = self._out(y_gla, y_swa, x)
        cache.state = state
        cache.put(kr, v, 0)
        cache.pos = x.shape[1]
        return out, cache

    @torch.no_grad()
    def step(self, hidden_states, position_embeddings, cache):
        """One token per sequence: hidden_states [B, 1, hidden] at position
        ``cache.pos`` (position_embeddings for that position, [B, 1, hd] or
        [1, hd]); updates ``cache`` in place and returns out [B, 1, hidden]."""
        x = hidden_states
        if x.dim() != 3 or x.shape[1] != 1:
            raise ValueError(f"LizardAttention.step: hidden_states must be [B, 1, hidden], got "
                             f"{tuple(x.shape)}")
        z, fq, fk, qr, kr, v = self._operands(x, position_embeddings)
        cache.put(kr, v, cache.pos)
        y_gla = kernels.gla_decode_step(fq[:, :, 0], fk[:, :, 0], v[:, :, 0], z[:, 0].contiguous(),
                                        cache.state, gate_logit=True)
        y_swa = kernels.swa_decode_step(qr[:, :, 0], cache.k, cache.v,
                                        self.meta_tokens.detach().float().contiguous(),
                                        cache.pos)
        cache.pos += 1
        return self._out(y_gla[:, :, None], y_swa[:, :, None], x)


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
