"""CPU oracle for the Lizard attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline).  The product (``lizard_reproduction_amd``) never imports it and
has no CPU fallback: without the HIP library it raises.

It restates, in plain PyTorch on the CPU, the math of the reference's dense
PyTorch functions (``src/lizard_attention.py:9-44`` of
mahdikhashan/lizard-reproduction) and the reference kernels' operator API
(``src/kernels/gla.py:259-263``, ``src/kernels/swa.py:182-183``), plus

* closed-form loop/recurrent versions of every formula (the reference's own
  ground truth, ``tests/test_lizard.py:22-69``), written from the formulas;
* a chunked restatement of the 64-token chunk algorithm the HIP kernels run
  (``src/kernels/gla.py:19-101`` conventions: gates measured from the chunk
  boundary, every absorbed factor <= 1), optionally emulating the bf16
  roundings of the kernel's MFMA operands.

How each function is pinned (all in ``tests/test_oracle.py``):

==================  =======================================================
function            pinned by
==================  =======================================================
window_mask         brute-force predicate on small sizes
gate_products       brute-force products; gla_loop / gla_recurrent
gla                 gla_loop, gla_recurrent (fp64, 1e-10); gate 0 -> v;
                    constant v stays constant; gate 1 -> normalised causal
                    linear attention; gradcheck
awa / sink_softmax  awa_loop (fp64, 1e-10); no sinks + huge window ==
                    torch SDPA(is_causal=True); many sinks == one logsumexp
                    sink; gradcheck
hedgehog            hedgehog_loop; halves are softmaxes (sum to one)
gla_kernel_api      gla on exp(log_gamma), per-head folding as the
                    reference's tests do (tests/test_kernels.py:61-70)
swa_kernel_api      awa; empty meta == meta of -1e4 (tests/test_kernels.py:
                    127-134)
gla_chunked         == dense gla in fp64 for chunk 16/64, L in {1,77,150},
                    per-token and per-head gates, strong decay
gla_recurrent_state outputs == gla_recurrent and dense gla (fp64); its state
                    == the chunked restatement's final state; S, z
                    decompose: fq_i S_i / fq_i z_i over i gives the outputs
rope                rope_loop; relative-position invariance of q.k
lizard_layer        lizard_layer_loop (fp64, 1e-10); with the GLA branch
                    zeroed, no sinks and an unbounded window it equals
                    transformers' LlamaAttention (a library routine);
                    causal and batch independent
awa_banded          == awa in fp64 for windows 1 .. > L, ragged L, block
                    sizes 16/64, empty meta, gradients included
lizard_layer_banded == lizard_layer in fp64 (output and every gradient) at
                    L <= 256, windows shorter and longer than a block
lizard_layer_       unrounded: == lizard_layer in fp64 (output and every
  rounded           gradient, fp32- and bf16-layer modes); rounded: each
                    rounding point moves the result (it is applied) and
                    stays within bf16 error of the unrounded layer; its
                    bf16 rounding is round-to-nearest-even (bf16 casts)
==================  =======================================================

The loops are deliberately independent code paths (explicit Python loops over
tokens), so a dropped term, a wrong sign, an off-by-one in the window or a
transposed operand in the vectorised functions fails a check.
"""
import math

import torch

TINY = torch.finfo(torch.float32).tiny


# ---------------------------------------------------------------------------
# Dense math (src/lizard_attention.py:9-44)
# ---------------------------------------------------------------------------

def hedgehog(x, weight):
    """Hedgehog feature map, ``src/lizard_attention.py:9-11``.

    phi(x) = [softmax(x W^T), softmax(-x W^T)] along the last dim, so the
    feature dimension is twice ``weight.shape[0]``.
    """
    proj = torch.matmul(x, weight.transpose(0, 1))
    return torch.cat([torch.softmax(proj, dim=-1),
                      torch.softmax(-proj, dim=-1)], dim=-1)


def window_mask(length, window, device=None):
    """Boolean [L, L] mask of the keys t a query i sees,
    ``src/lizard_attention.py:14-17``: t <= i and i - t < window (so the
    window holds ``window`` keys including the query itself)."""
    rows = torch.arange(length, device=device).unsqueeze(1)
    cols = torch.arange(length, device=device).unsqueeze(0)
    return (cols <= rows) & ((rows - cols) < window)


def gate_products(gamma):
    """Decay matrix D[..., i, t] = prod_{s=t+1..i} gamma_s for t <= i, else 0.

    Follows ``src/lizard_attention.py:20-25``: it works on gamma itself (not
    log gamma), so gamma == 0 is exact.  For row i the factors
    u_i[s] = gamma_s (s <= i) or 1 (s > i) are multiplied over s > t with a
    suffix product.
    """
    length = gamma.shape[-1]
    causal = window_mask(length, length, gamma.device)
    factors = torch.where(causal, gamma.unsqueeze(-2), torch.ones((), dtype=gamma.dtype))
    # inclusive suffix product over s >= t, then shift by one to get s > t
    suffix = torch.flip(torch.cumprod(torch.flip(factors, [-1]), dim=-1), [-1])
    exclusive = torch.cat([suffix[..., 1:], torch.ones_like(suffix[..., :1])], dim=-1)
    return exclusive * causal


def gla(fq, fk, v, gamma):
    """Dense gated linear attention, ``src/lizard_attention.py:28-31``.

    fq, fk: [B, H, L, F]; v: [B, H, L, D]; gamma: [B, L] (shared by heads).
    y_i = sum_t w_it v_t / max(sum_t w_it, tiny), w_it = (fq_i . fk_t) D_it.
    """
    weights = torch.matmul(fq, fk.transpose(-1, -2)) * gate_products(gamma).unsqueeze(1)
    tiny = torch.finfo(weights.dtype).tiny
    return torch.matmul(weights, v) / weights.sum(-1, keepdim=True).clamp_min(tiny)


def sink_softmax(scores, meta):
    """Softmax over the last dim with learned sink logits in the denominator
    only, ``src/lizard_attention.py:34-38``.  The shift m (row max, also over
    the sinks) is detached, as in the reference.  ``meta`` may be empty."""
    m = scores.amax(-1, keepdim=True)
    if meta.numel():
        m = torch.maximum(m, meta.max())
    m = m.detach()
    e = torch.exp(scores - m)
    den = e.sum(-1, keepdim=True)
    if meta.numel():
        den = den + torch.exp(meta - m).sum(-1, keepdim=True)
    return e / den


def awa(q, k, v, meta, window):
    """Dense sliding-window softmax with sinks, ``src/lizard_attention.py:41-44``.
    Scores are scaled by 1/sqrt(head_dim) and masked to the window."""
    mask = window_mask(q.shape[-2], window, q.device)
    scores = torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    scores = scores.masked_fill(~mask, float("-inf"))
    return torch.matmul(sink_softmax(scores, meta), v)


# ---------------------------------------------------------------------------
# Kernel operator API semantics (src/kernels/gla.py:259-263, swa.py:182-183)
# ---------------------------------------------------------------------------

def gla_kernel_api(fq, fk, v, log_gamma, dtype=torch.float32):
    """What ``kernels.gla(fq, fk, v, log_gamma)`` computes, in ``dtype``.

    log_gamma is [B, L] (one gate per token, shared by heads) or [B, H, L]
    (one gate per head); gamma = exp(log_gamma).  Per-head gates fold B*H into
    the batch, as the reference's tests do (``tests/test_kernels.py:61-70``).
    """
    batch, heads, length, _ = fq.shape
    gamma = torch.exp(log_gamma.to(dtype))
    if log_gamma.dim() == 2:
        return gla(fq.to(dtype), fk.to(dtype), v.to(dtype), gamma)

    def fold(t):
        return t.to(dtype).reshape(batch * heads, 1, length, -1)
    y = gla(fold(fq), fold(fk), fold(v), gamma.reshape(batch * heads, length))
    return y.reshape(batch, heads, length, -1)


def swa_kernel_api(q, k, v, meta, window, dtype=torch.float32):
    """What ``kernels.swa(q, k, v, meta, window)`` computes, in ``dtype``."""
    return awa(q.to(dtype), k.to(dtype), v.to(dtype), meta.to(dtype), window)


# ---------------------------------------------------------------------------
# Closed forms (tests/test_lizard.py:22-69), written as explicit loops
# ---------------------------------------------------------------------------

def hedgehog_loop(x, weight):
    proj = x @ weight.T
    pos, neg = torch.exp(proj), torch.exp(-proj)
    return torch.cat([pos / pos.sum(-1, keepdim=True),
                      neg / neg.sum(-1, keepdim=True)], dim=-1)


def gla_loop(fq, fk, v, gamma):
    """y_i = sum_{t<=i} w_it v_t / sum_{t<=i} w_it with
    w_it = (fq_i . fk_t) * prod_{s=t+1..i} gamma_s; gamma is [B, L]."""
    out = torch.zeros_like(v)
    for i in range(fq.shape[2]):
        num = torch.zeros_like(v[:, :, 0])
        den = torch.zeros_like(v[:, :, 0, :1])
        for t in range(i + 1):
            decay = torch.ones_like(gamma[:, 0])
            for s in range(t + 1, i + 1):
                decay = decay * gamma[:, s]
            w = decay[:, None, None] * (fq[:, :, i] * fk[:, :, t]).sum(-1, keepdim=True)
            num = num + w * v[:, :, t]
            den = den + w
        out[:, :, i] = num / den
    return out


def gla_recurrent(fq, fk, v, gamma):
    """Recurrent form: S_i = gamma_i S_{i-1} + fk_i v_i^T, z_i = gamma_i z_{i-1}
    + fk_i, y_i = fq_i S_i / (fq_i . z_i)."""
    b, h, n, f = fq.shape
    state = torch.zeros(b, h, f, v.shape[-1], dtype=fq.dtype)
    norm = torch.zeros(b, h, f, dtype=fq.dtype)
    outs = []
    for i in range(n):
        g = gamma[:, i].view(b, 1, 1)
        state = g[..., None] * state + fk[:, :, i, :, None] * v[:, :, i, None, :]
        norm = g * norm + fk[:, :, i]
        num = (fq[:, :, i, :, None] * state).sum(-2)
        outs.append(num / (fq[:, :, i] * norm).sum(-1, keepdim=True))
    return torch.stack(outs, dim=2)


def gla_recurrent_state(fq, fk, v, gamma):
    """The recurrent form of ``gla_recurrent`` returning also the state after
    the last token: (out, S [B, H, F, D], z [B, H, F]).  gamma is [B, L]
    (shared by heads) or [B, H, L]."""
    b, h, n, f = fq.shape
    state = torch.zeros(b, h, f, v.shape[-1], dtype=fq.dtype)
    norm = torch.zeros(b, h, f, dtype=fq.dtype)
    outs = []
    for i in range(n):
        g = gamma[..., i]
        g = g.view(b, 1, 1) if g.dim() == 1 else g.view(b, h, 1)
        state = g[..., None] * state + fk[:, :, i, :, None] * v[:, :, i, None, :]
        norm = g * norm + fk[:, :, i]
        num = (fq[:, :, i, :, None] * state).sum(-2)
        den = (fq[:, :, i] * norm).sum(-1, keepdim=True)
        outs.append(num / den.clamp_min(TINY))
    return torch.stack(outs, dim=2), state, norm


def awa_loop(q, k, v, meta, window):
    """y_i = sum_{i-W<t<=i} e^{s_it} v_t / (sum_j e^{meta_j} + sum_t e^{s_it}),
    s_it = q_i . k_t / sqrt(d)."""
    out = torch.zeros_like(v)
    for i in range(q.shape[2]):
        lo = max(0, i - window + 1)
        scores = (q[:, :, i, None] * k[:, :, lo:i + 1]).sum(-1) / math.sqrt(q.shape[-1])
        e = torch.exp(scores)
        num = (e[..., None] * v[:, :, lo:i + 1]).sum(-2)
        sinks = meta.exp().sum() if meta.numel() else 0.0
        out[:, :, i] = num / (sinks + e.sum(-1, keepdim=True))
    return out


def rope_loop(x, cos, sin):
    """rotate_half RoPE: x*cos + [-x2, x1]*sin, cos/sin [L, d]."""
    half = x.shape[-1] // 2
    out = torch.empty_like(x)
    for j in range(x.shape[-1]):
        partner = -x[..., j + half] if j < half else x[..., j - half]
        out[..., j] = x[..., j] * cos[:, j] + partner * sin[:, j]
    return out


def rope_cos_sin(length, dim, theta=500000.0, dtype=torch.float64):
    """Default (unscaled) RoPE tables [L, d] with the rotate_half convention,
    as transformers' Llama rotary embedding builds them."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    pos = torch.arange(length, dtype=torch.float64)
    ang = torch.outer(pos, inv)
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rope(x, cos, sin):
    """Vectorised rotate_half RoPE, pinned by ``rope_loop``."""
    half = x.shape[-1] // 2
    rotated = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rotated * sin


# ---------------------------------------------------------------------------
# Chunked restatement of the kernel algorithm (src/kernels/gla.py:19-101)
# ---------------------------------------------------------------------------

def _bf16(t):
    return t.to(torch.bfloat16).to(t.dtype)


def gla_chunked(fq, fk, v, log_gamma, chunk=64, round_bf16=False, dtype=torch.float64,
                return_state=False):
    """Chunkwise GLA with gates measured from each chunk's boundary.

    Within chunk n (tokens [nC, nC+C)), lg_j is the inclusive sum of
    log_gamma over the chunk up to token j, lg_end its last value:

    * Q~_i = fq_i exp(lg_i) and K~_t = fk_t exp(lg_end - lg_t)  (both <= 1);
    * o_i = Q~_i S_n + sum_{t<=i} a_it v_t, a_it = (fq_i . fk_t) exp(lg_i - lg_t);
    * den_i = Q~_i . z_n + sum_{t<=i} a_it;  y_i = o_i / max(den_i, tiny);
    * S_{n+1} = exp(lg_end) S_n + K~^T V,  z_{n+1} = exp(lg_end) z_n + sum_t K~_t.

    The reference measures the same differences from a global cumsum
    (start = G[nC-1], end = G[last]); here they are chunk-local sums, which is
    what the HIP kernels do.  With ``round_bf16`` the kernel's bf16 MFMA
    operands (K~, a and the state used by Q~ S) are rounded as the kernel
    rounds them; Q~ stays unrounded, as in the kernel, which applies the row
    scale exp(lg_i) to the fp32 products fq . S and fq . z.
    log_gamma: [B, L] or [B, H, L].  Returns [B, H, L, D]; with
    ``return_state`` also the state after the last token (S [B, H, F, D],
    z [B, H, F]).
    """
    batch, heads, length, nf = fq.shape
    nd = v.shape[-1]
    fq, fk, v = fq.to(dtype), fk.to(dtype), v.to(dtype)
    lgam = log_gamma.to(dtype)
    if lgam.dim() == 2:
        lgam = lgam[:, None, :].expand(batch, heads, length)
    rnd = _bf16 if round_bf16 else (lambda t: t)
    state = torch.zeros(batch, heads, nf, nd, dtype=dtype)
    norm = torch.zeros(batch, heads, nf, dtype=dtype)
    outs = []
    # chunks by split and outputs joined by cat, so that autograd's backward
    # stays linear in L (a slice's backward would fill a whole-length buffer)
    if length == 0:
        outs.append(torch.empty(batch, heads, 0, nd, dtype=dtype))
    pieces = (torch.split(t, chunk, dim=2) for t in (fq, fk, v))
    for q, k, vv, lgc in zip(*pieces, torch.split(lgam, chunk, dim=-1)):
        lg = torch.cumsum(lgc, dim=-1)                         # [B,H,c]
        lg_end = lg[..., -1:]
        qt = q * torch.exp(lg)[..., None]
        kt = rnd(k * torch.exp(lg_end - lg)[..., None])
        n = q.shape[2]
        causal = torch.ones(n, n, dtype=torch.bool).tril()
        diff = lg[..., :, None] - lg[..., None, :]
        decay = torch.exp(torch.where(causal, diff, torch.full_like(diff, -math.inf)))
        a = rnd(torch.matmul(q, k.transpose(-1, -2)) * decay)
        o = torch.matmul(qt, rnd(state)) + torch.matmul(a, vv)
        den = (qt * norm[:, :, None, :]).sum(-1) + a.sum(-1)
        outs.append(o / den.clamp_min(TINY)[..., None])
        r = torch.exp(lg_end)[..., None]                       # [B,H,1,1]
        state = state * r + torch.matmul(kt.transpose(-1, -2), vv)
        norm = norm * r[..., 0] + kt.sum(-2)
    out = torch.cat(outs, dim=2)
    if return_state:
        return out, state, norm
    return out


# ---------------------------------------------------------------------------
# The whole attention layer (src/lizard_attention.py:47-97)
# ---------------------------------------------------------------------------

def lizard_layer(params, x, cos, sin, heads, kv_heads, window):
    """Dense ``LizardAttention.forward`` of the reference's torch backend,
    ``src/lizard_attention.py:73-97``, on a dict of its parameters (names as
    ``named_parameters()`` gives them).

    x [B, L, hidden]; cos, sin [B, L, head_dim] (transformers' rotary tables,
    broadcast over heads as ``apply_rotary_pos_emb`` does with unsqueeze_dim
    1).  Projections run in x's dtype, everything after them in
    promote(x.dtype, fp32); heads are expanded from the kv heads by
    repeat_interleave; y = gla(phi_q(q), phi_k(k), v, sigmoid(z)) +
    alpha * awa(rope(q), rope(k), v, meta, window); out = o_proj(y).
    """
    batch, length, hidden = x.shape
    head_dim = hidden // heads
    dtype = torch.promote_types(x.dtype, torch.float32)

    def heads_of(name, count):
        y = torch.matmul(x, params[name].transpose(0, 1)).view(batch, length, count, head_dim)
        return y.transpose(1, 2).repeat_interleave(heads // count, dim=1).to(dtype)

    q = heads_of("q_proj.weight", heads)
    k = heads_of("k_proj.weight", kv_heads)
    v = heads_of("v_proj.weight", kv_heads)
    z = torch.matmul(x, params["W_gamma.weight"].transpose(0, 1)).to(dtype).squeeze(-1)
    fq = hedgehog(q, params["phi_q.weight"].to(dtype))
    fk = hedgehog(k, params["phi_k.weight"].to(dtype))
    c, s = cos.to(dtype).unsqueeze(1), sin.to(dtype).unsqueeze(1)
    qr, kr = rope(q, c, s), rope(k, c, s)
    alpha, meta = params["alpha_blend"].to(dtype), params["meta_tokens"].to(dtype)
    y = gla(fq, fk, v, torch.sigmoid(z)) + alpha * awa(qr, kr, v, meta, window)
    y = y.to(x.dtype).transpose(1, 2).reshape(batch, length, hidden)
    return torch.matmul(y, params["o_proj.weight"].transpose(0, 1))


class _RoundBF16(torch.autograd.Function):
    """bf16 rounding of a value (kept in its dtype) whose gradient is rounded
    the same way on the way back: what a bf16 tensor between two HIP kernels
    does to both (autograd hands a bf16 output a bf16 upstream gradient)."""

    @staticmethod
    def forward(ctx, x):
        return x.to(torch.bfloat16).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def round_bf16(t):
    """``_RoundBF16`` applied to t."""
    return _RoundBF16.apply(t)


def lizard_layer_rounded(params, x, cos, sin, heads, kv_heads, window, rounded=True,
                         bf16_layer=False, chunk=64):
    """``lizard_layer`` in x's dtype (fp64 for a checker) with the bf16
    rounding points of the HIP layer, forward and backward: the model of what
    bf16 operands do to the layer, against which the HIP layer's output and
    gradients are compared directly.

    Rounding points (all with ``rounded``; none without, which leaves the
    reference's layer, src/lizard_attention.py:73-97):

    * the kernel operands fq, fk, rotated q and k, and v, and the two branch
      outputs (the fused layer hands them over in bf16, both ways:
      ``round_bf16``);
    * inside the GLA branch, the chunked algorithm's bf16 MFMA operands
      (``gla_chunked(round_bf16=True)``: K~, the weights a, the state used
      by Q~ S), their gradients rounded the same way under autograd;
    * inside the SWA branch, the probabilities P before P V in the forward
      (the kernel's bf16 MFMA operand; ``awa_banded(round_p=True)``);
    * with ``bf16_layer`` (a layer whose parameters and input are bf16):
      the projection outputs q, k, v and the gate logit (torch's bf16
      GEMMs), the blended y before o_proj, and the layer's output.

    The GLA branch is ``gla_chunked`` on log_gamma = logsigmoid(z), the SWA
    branch ``awa_banded``: unrounded, both equal the dense forms in fp64, so
    long L fits.  cos, sin [B, L, hd] or [L, hd]."""
    batch, length, hidden = x.shape
    head_dim = hidden // heads
    r = round_bf16 if rounded else (lambda t: t)
    rp = r if bf16_layer else (lambda t: t)

    def heads_of(name, count):
        y = rp(torch.matmul(x, params[name].transpose(0, 1)))
        y = y.view(batch, length, count, head_dim).transpose(1, 2)
        return y.repeat_interleave(heads // count, dim=1)

    q = heads_of("q_proj.weight", heads)
    k = heads_of("k_proj.weight", kv_heads)
    v = heads_of("v_proj.weight", kv_heads)
    z = rp(torch.matmul(x, params["W_gamma.weight"].transpose(0, 1))).squeeze(-1)
    fq, fk = hedgehog(q, params["phi_q.weight"]), hedgehog(k, params["phi_k.weight"])
    c, s = cos.to(x.dtype), sin.to(x.dtype)
    c, s = (c if c.dim() == 3 else c[None]).unsqueeze(1), (s if s.dim() == 3 else s[None]).unsqueeze(1)
    qr, kr = rope(q, c, s), rope(k, c, s)
    y_gla = r(gla_chunked(r(fq), r(fk), r(v), torch.nn.functional.logsigmoid(z), chunk,
                          round_bf16=rounded, dtype=x.dtype))
    y_swa = r(awa_banded(r(qr), r(kr), r(v), params["meta_tokens"], window, round_p=rounded))
    y = rp(y_gla + params["alpha_blend"] * y_swa)
    y = y.transpose(1, 2).reshape(batch, length, hidden)
    return rp(torch.matmul(y, params["o_proj.weight"].transpose(0, 1)))


def awa_banded(q, k, v, meta, window, block=64, round_p=False):
    """``awa`` computed block by block over the queries, each block against
    only the keys its window can reach (keys i0 - window + 1 .. i1 - 1 for
    queries i0 .. i1 - 1), so memory is O(L (block + window)) instead of
    O(L^2): the long-L form of the dense SWA oracle.  Same mask
    (``window_mask``'s predicate), scale and ``sink_softmax``.  With
    ``round_p`` the probabilities are rounded to bf16 before P V (the SWA
    forward's MFMA operand) in the forward only: the gradient passes
    unrounded, as the SWA backward recomputes P in fp32 for delta and the
    sink gradient."""
    length, dim = q.shape[-2], q.shape[-1]
    if length == 0:
        return torch.empty_like(v)
    # blocks by split and the keys a block reaches by cat, so that autograd's
    # backward stays linear in L (a slice of the whole k would fill a
    # whole-length buffer in its backward)
    qb, kb, vb = (torch.split(t, block, dim=-2) for t in (q, k, v))
    outs = []
    for n, qq in enumerate(qb):
        i0 = n * block
        i1 = i0 + qq.shape[-2]
        t0 = max(0, i0 - window + 1)
        first = t0 // block
        kk = torch.cat(kb[first:n + 1], dim=-2)[..., t0 - first * block:, :]
        vv = torch.cat(vb[first:n + 1], dim=-2)[..., t0 - first * block:, :]
        rows = torch.arange(i0, i1).unsqueeze(1)
        cols = torch.arange(t0, i1).unsqueeze(0)
        mask = (cols <= rows) & ((rows - cols) < window)
        scores = torch.matmul(qq, kk.transpose(-1, -2))
        scores = (scores / math.sqrt(dim)).masked_fill(~mask, float("-inf"))
        p = sink_softmax(scores, meta)
        if round_p:
            p = p + (p.detach().to(torch.bfloat16).to(p.dtype) - p.detach())
        outs.append(torch.matmul(p, vv))
    return torch.cat(outs, dim=-2)


def lizard_layer_banded(params, x, cos, sin, heads, kv_heads, window, chunk=64):
    """``lizard_layer`` with its two O(L^2) pieces replaced by their long-L
    forms: the GLA branch by ``gla_chunked`` on log_gamma = logsigmoid(z)
    (exact in fp64, no rounding), the SWA branch by ``awa_banded``.  Same
    projections, dtype promotion, repeat_interleave GQA expansion, Hedgehog
    maps, RoPE and blend (``src/lizard_attention.py:73-97``).  Pinned against
    ``lizard_layer`` at lengths the dense form holds; it is the oracle of the
    layer at BASELINE config 5's sequence length."""
    batch, length, hidden = x.shape
    head_dim = hidden // heads
    dtype = torch.promote_types(x.dtype, torch.float32)

    def heads_of(name, count):
        y = torch.matmul(x, params[name].transpose(0, 1)).view(batch, length, count, head_dim)
        return y.transpose(1, 2).repeat_interleave(heads // count, dim=1).to(dtype)

    q = heads_of("q_proj.weight", heads)
    k = heads_of("k_proj.weight", kv_heads)
    v = heads_of("v_proj.weight", kv_heads)
    z = torch.matmul(x, params["W_gamma.weight"].transpose(0, 1)).to(dtype).squeeze(-1)
    fq = hedgehog(q, params["phi_q.weight"].to(dtype))
    fk = hedgehog(k, params["phi_k.weight"].to(dtype))
    c, s = cos.to(dtype).unsqueeze(1), sin.to(dtype).unsqueeze(1)
    qr, kr = rope(q, c, s), rope(k, c, s)
    alpha, meta = params["alpha_blend"].to(dtype), params["meta_tokens"].to(dtype)
    y_gla = gla_chunked(fq, fk, v, torch.nn.functional.logsigmoid(z), chunk, dtype=dtype)
    y = y_gla + alpha * awa_banded(qr, kr, v, meta, window)
    y = y.to(x.dtype).transpose(1, 2).reshape(batch, length, hidden)
    return torch.matmul(y, params["o_proj.weight"].transpose(0, 1))


def lizard_layer_loop(params, x, cos, sin, heads, kv_heads, window):
    """The same layer composed from the closed-form loops (hedgehog_loop,
    gla_loop, awa_loop, rope_loop), with the kv-head expansion written as an
    explicit index map (head h reads kv head h // (heads / kv_heads)).  The
    reference's own ground truth for its layer is this composition
    (tests/test_lizard.py:72-91).  cos, sin [L, head_dim]."""
    batch, length, hidden = x.shape
    head_dim = hidden // heads
    group = heads // kv_heads

    def project(name, count):
        w = params[name]
        out = torch.empty(batch, heads, length, head_dim, dtype=x.dtype)
        for h in range(heads):
            src = h if count == heads else h // group
            rows = w[src * head_dim:(src + 1) * head_dim]
            out[:, h] = torch.matmul(x, rows.transpose(0, 1))
        return out

    q, k, v = (project(n, c) for n, c in (("q_proj.weight", heads),
                                          ("k_proj.weight", kv_heads),
                                          ("v_proj.weight", kv_heads)))
    gamma = 1.0 / (1.0 + torch.exp(-torch.matmul(x, params["W_gamma.weight"][0])))
    fq = hedgehog_loop(q, params["phi_q.weight"])
    fk = hedgehog_loop(k, params["phi_k.weight"])
    qr, kr = rope_loop(q, cos, sin), rope_loop(k, cos, sin)
    y = gla_loop(fq, fk, v, gamma) + params["alpha_blend"] * awa_loop(
        qr, kr, v, params["meta_tokens"], window)
    y = y.transpose(1, 2).reshape(batch, length, hidden)
    return torch.matmul(y, params["o_proj.weight"].transpose(0, 1))
