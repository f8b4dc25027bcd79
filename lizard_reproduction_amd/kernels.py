"""Operator API of the Lizard attention hot path on MI355X (gfx950).

Drop-in for the reference's ``kernels`` package (``src/kernels/__init__.py``):

* ``gla(fq, fk, v, log_gamma, chunk=64)``  -- ``src/kernels/gla.py:259-263``
* ``swa(q, k, v, meta, window, fwd_blocks=(64, 64), bwd_blocks=(64, 64))``
  -- ``src/kernels/swa.py:182-183``

Same signatures, shapes and conventions: tensors are ``[B, H, L, .]``; inputs
of any float dtype are cast to bf16; outputs are bf16; gradients come back in
each input's dtype; the gate is ``[B, L]`` (one per token, shared by heads) or
``[B, H, L]`` (one per head).  ``chunk`` and ``*_blocks`` are tiling hints in
the reference; results do not depend on them beyond rounding, and the HIP
kernels always use their own tiles (64-token GLA chunks, 32-row SWA tiles).

Every call goes through the C ABI of ``liblizard_hip.so`` on the current HIP
stream; there is no CPU or PyTorch fallback.
"""
import functools
import math

import torch

from . import _lib

CHUNK = 64
FWD_BLOCKS = (64, 64)
BWD_BLOCKS = (64, 64)


def _stream(t):
    """Raw hipStream_t of the current stream of t's device (launches go there,
    as the reference's Triton launches go to torch's current stream)."""
    try:
        return torch._C._cuda_getCurrentRawStream(t.device.index)
    except AttributeError:   # pragma: no cover - older torch without the raw accessor
        return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None and t.numel() else None


@functools.lru_cache(maxsize=256)
def _gla_fwd_ws(b, h, length, nf, nd, per_head, chunk):
    return _lib.load().lz_gla_fwd_workspace_bytes(b, h, length, nf, nd, per_head, chunk)


@functools.lru_cache(maxsize=256)
def _gla_bwd_ws(b, h, length, nf, nd, per_head, chunk):
    return _lib.load().lz_gla_bwd_workspace_bytes(b, h, length, nf, nd, per_head, chunk)


@functools.lru_cache(maxsize=256)
def _swa_bwd_ws(b, h, length, d, n_meta):
    return _lib.load().lz_swa_bwd_workspace_bytes(b, h, length, d, n_meta)


def _refuse_capture(what):
    """Refuse calls made while the current stream is being captured into a
    HIP graph.  The wrappers allocate outputs and workspaces with torch on
    every call, and the library sets a kernel's LDS limit with
    hipFuncSetAttribute on its first launch on a device; a capture of a
    whole fwd+bwd crashed the host process once (in the runtime's capture
    end) and neither step has been cleared as its cause, so capture is not
    offered."""
    if _gpu_present() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"{what}: calls under HIP graph capture are not supported "
                           "(run the kernels eagerly)")


_GPU_SEEN = False


def _gpu_present():
    """torch.cuda.is_available(), remembered once true (it is asked on every
    launch, and the query costs about a microsecond of host time)."""
    global _GPU_SEEN
    if not _GPU_SEEN:
        _GPU_SEEN = torch.cuda.is_available()
    return _GPU_SEEN


def _require_gpu(*tensors):
    _refuse_capture("lizard_reproduction_amd kernels")
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("lizard_reproduction_amd kernels need tensors on a ROCm GPU "
                             f"(got a tensor on {t.device})")


# The casts below return their input unchanged when it already has the
# dtype and layout (the common case): a dtype/contiguity test is far cheaper
# per call than .to(...).contiguous(), and these wrappers run once per launch.
def _bf16(t):
    if t.dtype is torch.bfloat16 and t.is_contiguous():
        return t
    return t.to(torch.bfloat16).contiguous()


def _f32(t):
    if t.dtype is torch.float32 and t.is_contiguous():
        return t
    return t.float().contiguous()


def _cast_grads(grads, dtypes):
    return tuple(g if g.dtype is d else g.to(d) for g, d in zip(grads, dtypes))


# ---------------------------------------------------------------------------
# gated linear attention
# ---------------------------------------------------------------------------

def _check_gla(fq, fk, v, log_gamma, chunk):
    if fq.dim() != 4 or fk.shape != fq.shape:
        raise ValueError(f"gla: fq and fk must be [B, H, L, F] of one shape, got "
                         f"{tuple(fq.shape)} and {tuple(fk.shape)}")
    if v.dim() != 4 or v.shape[:3] != fq.shape[:3]:
        raise ValueError(f"gla: v must be [B, H, L, D] matching fq, got {tuple(v.shape)}")
    b, h, length, _ = fq.shape
    if tuple(log_gamma.shape) not in ((b, length), (b, h, length)):
        raise ValueError(f"gla: log_gamma must be [B, L] or [B, H, L], got "
                         f"{tuple(log_gamma.shape)} for fq {tuple(fq.shape)}")
    if not isinstance(chunk, int) or chunk < 16 or chunk & (chunk - 1):
        raise ValueError(f"gla: chunk must be a power of two >= 16, got {chunk!r}")
    _require_gpu(fq, fk, v, log_gamma)


def _check_kv(what, q, k, v, nk, nv):
    """Shapes of the internal launch wrappers: q [B, H, L, nk]; k [B, Hkv,
    L, nk] and v [B, Hkv, L, nv] with Hkv dividing H (the kernels index the
    buffers from these sizes alone)."""
    b, h, length = q.shape[:3]
    hk = k.shape[1] if k.dim() == 4 else 0
    if q.dim() != 4 or q.shape[3] != nk or tuple(k.shape) != (b, hk, length, nk) or \
            tuple(v.shape) != (b, hk, length, nv) or hk <= 0 or h % hk:
        raise ValueError(f"{what}: need q [B, H, L, {nk}], k [B, Hkv, L, {nk}], "
                         f"v [B, Hkv, L, {nv}] with Hkv dividing H; got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")


def _check_gate(what, fq, lg):
    b, h, length = fq.shape[:3]
    if tuple(lg.shape) not in ((b, length), (b, h, length)):
        raise ValueError(f"{what}: log_gamma must be {(b, length)} or {(b, h, length)}, "
                         f"got {tuple(lg.shape)}")


def _padded(n):
    return next((p for p in (32, 64, 128, 256) if n <= p), None)


def gla_native(nf, nd):
    """Whether the GLA walks take (F, D) directly (F <= 256, D <= 128, D <= 64
    when F > 128); past that the library runs them on tiles, and the
    forward's workspace holds tiles rather than segment states."""
    fp, dp = _padded(nf), _padded(nd)
    return fp is not None and dp is not None and dp <= 128 and (fp <= 128 or dp <= 64)


# gate_mode bits of the C ABI (include/lizard_hip.h)
GATE_PER_HEAD, GATE_LOGIT, GLA_NO_REUSE = 1, 2, 4


def _gate_mode(lg, gate_logit):
    return (GATE_PER_HEAD if lg.dim() == 3 else 0) | (GATE_LOGIT if gate_logit else 0)


def gla_forward(fq, fk, v, lg, keep_state=True, chunk=CHUNK, gate_logit=False):
    """One ``lz_gla_fwd`` launch on bf16 contiguous fq, fk, v and fp32
    contiguous log_gamma; returns (y, state), state being the workspace of
    the sequence segments' state records, which ``gla_backward`` reuses
    (None when not kept, not needed, or for tiled sizes past the walks').
    Not keeping it also tells the kernels that nothing reads fq, fk, v again
    soon (``LZ_GLA_NO_REUSE``: no backward follows).  fk and v may have fewer heads than
    fq (a divisor: grouped-query attention, each kv head shared by
    consecutive query heads).  With ``gate_logit`` lg holds the gate's logit
    z and the kernels use log_gamma = logsigmoid(z) (the layer's
    F.logsigmoid, src/lizard_attention.py:92)."""
    _check_kv("gla_forward", fq, fk, v, fq.shape[-1], v.shape[-1])
    _check_gate("gla_forward", fq, lg)
    return _gla_fwd_launch(fq, fk, v, lg, keep_state, chunk, gate_logit)


def _gla_fwd_launch(fq, fk, v, lg, keep_state, chunk, gate_logit):
    """``gla_forward`` without its shape checks (for callers that made them)."""
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    y = torch.empty(b, h, length, nd, device=v.device, dtype=v.dtype)
    ws = None
    if y.numel():
        lib = _lib.load()
        mode = _gate_mode(lg, gate_logit) | (0 if keep_state else GLA_NO_REUSE)
        nbytes = _gla_fwd_ws(b, h, length, nf, nd, mode & GATE_PER_HEAD, chunk)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=fq.device) if nbytes else None
        rc = lib.lz_gla_fwd(_ptr(fq), _ptr(fk), _ptr(v), _ptr(lg), _ptr(y), b, h, fk.shape[1],
                            length, nf, nd, mode, chunk, _ptr(ws), nbytes, _stream(fq))
        _lib.check(rc, "lz_gla_fwd")
    return y, (ws if keep_state and gla_native(nf, nd) else None)


def gla_backward(fq, fk, v, lg, dy, state, grad_dtype, chunk=CHUNK, gate_logit=False):
    """One ``lz_gla_bwd`` launch: (dfq, dfk, dv) in grad_dtype (bf16 or
    fp32) and dlog_gamma fp32 in log_gamma's layout (with ``gate_logit``,
    the gradient of the logit lg holds).  dfk and dv are per query head,
    also when fk and v have fewer (kv) heads."""
    _check_kv("gla_backward", fq, fk, v, fq.shape[-1], v.shape[-1])
    _check_gate("gla_backward", fq, lg)
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    if tuple(dy.shape) != (b, h, length, nd):
        raise ValueError(f"gla_backward: dy must be {(b, h, length, nd)}, got {tuple(dy.shape)}")
    return _gla_bwd_launch(fq, fk, v, lg, dy, state, grad_dtype, chunk, gate_logit)


def _gla_bwd_launch(fq, fk, v, lg, dy, state, grad_dtype, chunk, gate_logit):
    """``gla_backward`` without its shape checks (for callers that made them)."""
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    dfq = torch.empty(fq.shape, device=fq.device, dtype=grad_dtype)
    dfk = torch.empty_like(dfq)
    dv = torch.empty(b, h, length, nd, device=v.device, dtype=grad_dtype)
    dlg = torch.empty_like(lg)
    if dy.numel():
        lib = _lib.load()
        mode = _gate_mode(lg, gate_logit)
        nbytes = _gla_bwd_ws(b, h, length, nf, nd, mode & GATE_PER_HEAD, chunk)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=fq.device)
        rc = lib.lz_gla_bwd(_ptr(fq), _ptr(fk), _ptr(v), _ptr(lg), _ptr(dy), _ptr(dfq),
                            _ptr(dfk), _ptr(dv), _ptr(dlg), int(grad_dtype == torch.bfloat16),
                            b, h, fk.shape[1], length, nf, nd, mode, chunk, _ptr(state),
                            state.numel() if state is not None else 0, _ptr(ws), ws.numel(),
                            _stream(fq))
        _lib.check(rc, "lz_gla_bwd")
    else:
        dfq.zero_(), dfk.zero_(), dv.zero_(), dlg.zero_()
    return dfq, dfk, dv, dlg


class _GLA(torch.autograd.Function):
    """Autograd node of ``gla``; mirrors ``_GLA`` (src/kernels/gla.py:213-256),
    but takes log_gamma itself: its cumsum, head expand and their gradients
    run inside the kernels."""

    @staticmethod
    def forward(ctx, fq, fk, v, log_gamma, chunk):
        ctx.dtypes = (fq.dtype, fk.dtype, v.dtype, log_gamma.dtype)
        fq, fk, v = _bf16(fq), _bf16(fk), _bf16(v)
        lg = _f32(log_gamma)
        grad = any(ctx.needs_input_grad[:4])
        y, state = _gla_fwd_launch(fq, fk, v, lg, grad, chunk, False)
        if grad:
            ctx.save_for_backward(fq, fk, v, lg)
            # the segments' state records, reused by the backward
            ctx.fwd_ws = state
        ctx.chunk = chunk
        return y

    @staticmethod
    def backward(ctx, dy):
        fq, fk, v, lg = ctx.saved_tensors
        gdt = torch.bfloat16 if all(d == torch.bfloat16 for d in ctx.dtypes[:3]) else torch.float32
        grads = _gla_bwd_launch(fq, fk, v, lg, _bf16(dy), ctx.fwd_ws, gdt, ctx.chunk, False)
        return _cast_grads(grads, ctx.dtypes) + (None,)


def gla_prefill(fq, fk, v, log_gamma, chunk=CHUNK, gate_logit=False):
    """``gla`` forward (no autograd) that also returns the recurrent state
    after the last token, for decoding: ``(y, state)``, state fp32
    ``[B, H, F*D + F]`` (S row-major ``[F][D]``, then z ``[F]``; see
    ``split_state``).  The reference has no decode path; the state is that of
    its recurrent form (tests/test_lizard.py:41-52).  fk and v may have fewer
    heads than fq (a divisor, as in ``gla_forward``); ``gate_logit`` as
    there."""
    if not isinstance(chunk, int) or chunk < 16 or chunk & (chunk - 1):
        raise ValueError(f"gla_prefill: chunk must be a power of two >= 16, got {chunk!r}")
    _check_kv("gla_prefill", fq, fk, v, fq.shape[-1], v.shape[-1])
    _check_gate("gla_prefill", fq, log_gamma)
    _require_gpu(fq, fk, v, log_gamma)
    fq, fk, v = _bf16(fq), _bf16(fk), _bf16(v)
    lg = _f32(log_gamma)
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    y = torch.empty(b, h, length, nd, device=v.device, dtype=torch.bfloat16)
    state = torch.zeros(b, h, nf * nd + nf, device=fq.device, dtype=torch.float32)
    if y.numel():
        lib = _lib.load()
        mode = _gate_mode(lg, gate_logit) | GLA_NO_REUSE   # inference: no backward
        nbytes = _gla_fwd_ws(b, h, length, nf, nd, mode & GATE_PER_HEAD, chunk)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=fq.device) if nbytes else None
        rc = lib.lz_gla_prefill(_ptr(fq), _ptr(fk), _ptr(v), _ptr(lg), _ptr(y), _ptr(state), b, h,
                                fk.shape[1], length, nf, nd, mode, chunk, _ptr(ws), nbytes,
                                _stream(fq))
        _lib.check(rc, "lz_gla_prefill")
    return y, state


def gla_forward_phi(qp, wq, fk, v, lg, heads, gate_logit=False, final_state=False,
                    chunk=CHUNK):
    """One ``lz_gla_fwd_phi`` launch: the GLA forward with fq formed inside
    the walk from the q projection rows and the feature weights --
    fq = [softmax(q Wq^T), softmax(-q Wq^T)] (src/lizard_attention.py:9-11)
    -- so fq never goes through memory.  qp bf16 ``[B, L, heads * 64]`` (the
    q_proj output), wq bf16 ``[128, 64]``, fk bf16 ``[B, Hkv, L, 256]``, v
    bf16 ``[B, Hkv, L, 64]``, lg as ``gla_forward`` (``gate_logit`` too).
    Returns (y bf16 ``[B, heads, L, 64]``, the recurrent state after the last
    token as ``gla_prefill`` returns it, or None)."""
    if qp.dim() != 3 or heads <= 0 or qp.shape[-1] != heads * 64 or tuple(wq.shape) != (128, 64):
        raise ValueError(f"gla_forward_phi: q [B, L, heads * 64] and wq [128, 64] expected, got "
                         f"{tuple(qp.shape)} ({heads} heads) and {tuple(wq.shape)}")
    b, length, _ = qp.shape
    hk = fk.shape[1] if fk.dim() == 4 else 0
    if tuple(fk.shape) != (b, hk, length, 256) or tuple(v.shape) != (b, hk, length, 64) or \
            hk <= 0 or heads % hk:
        raise ValueError(f"gla_forward_phi: fk [B, Hkv, L, 256] and v [B, Hkv, L, 64] with Hkv "
                         f"dividing {heads} expected, got {tuple(fk.shape)}, {tuple(v.shape)}")
    if tuple(lg.shape) not in ((b, length), (b, heads, length)):
        raise ValueError(f"gla_forward_phi: log_gamma must be {(b, length)} or "
                         f"{(b, heads, length)}, got {tuple(lg.shape)}")
    _require_gpu(qp, wq, fk, v, lg)
    for name, t in (("q", qp), ("wq", wq), ("fk", fk), ("v", v)):
        if t.dtype is not torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"gla_forward_phi: {name} must be contiguous bf16")
    lg = _f32(lg)
    y = torch.empty(b, heads, length, 64, device=qp.device, dtype=torch.bfloat16)
    state = new_state(b, heads, 256, 64, qp.device) if final_state else None
    if y.numel():
        mode = _gate_mode(lg, gate_logit)
        nbytes = _gla_fwd_ws(b, heads, length, 256, 64, mode & GATE_PER_HEAD, chunk)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=qp.device) if nbytes else None
        rc = _lib.load().lz_gla_fwd_phi(_ptr(qp), _ptr(wq), _ptr(fk), _ptr(v), _ptr(lg), _ptr(y),
                                        _ptr(state), b, heads, hk, length, 64, 128, mode, chunk,
                                        _ptr(ws), nbytes, _stream(qp))
        _lib.check(rc, "lz_gla_fwd_phi")
    return y, state


def new_state(batch, heads, nf, nd, device):
    """The recurrent state of an empty prefix (zeros), ``[B, H, F*D + F]`` fp32."""
    return torch.zeros(batch, heads, nf * nd + nf, device=device, dtype=torch.float32)


def split_state(state, nf, nd):
    """Views (S ``[B, H, F, D]``, z ``[B, H, F]``) of a recurrent state."""
    b, h, _ = state.shape
    return state[..., :nf * nd].view(b, h, nf, nd), state[..., nf * nd:]


def gla_decode_step(fq, fk, v, log_gamma, state, gate_logit=False):
    """One token per (b, h) on the recurrent form, updating ``state`` in place
    (tests/test_lizard.py:41-52): S <- gamma S + fk v^T, z <- gamma z + fk,
    y = fq S / max(fq . z, FLT_MIN), gamma = exp(log_gamma).

    fq ``[B, H, F]``, fk ``[B, Hkv, F]``, v ``[B, Hkv, D]`` (cast to bf16;
    Hkv divides H, query head h reads kv head h // (H // Hkv)), log_gamma
    ``[B]`` or ``[B, H]`` fp32 (with ``gate_logit`` the gate's logit z,
    log_gamma = logsigmoid(z)), state from ``gla_prefill`` or ``new_state``.
    Returns bf16 ``[B, H, D]``; no autograd."""
    if fq.dim() != 3 or fk.dim() != 3 or v.dim() != 3:
        raise ValueError(f"gla_decode_step: fq [B, H, F], fk [B, Hkv, F] and v [B, Hkv, D] "
                         f"expected, got {tuple(fq.shape)}, {tuple(fk.shape)}, {tuple(v.shape)}")
    b, h, nf = fq.shape
    nd = v.shape[-1]
    hk = fk.shape[1]
    if tuple(fk.shape) != (b, hk, nf) or tuple(v.shape) != (b, hk, nd) or hk <= 0 or h % hk:
        raise ValueError(f"gla_decode_step: fq [B, H, F], fk [B, Hkv, F] and v [B, Hkv, D] with "
                         f"Hkv dividing H expected, got {tuple(fq.shape)}, {tuple(fk.shape)}, "
                         f"{tuple(v.shape)}")
    if log_gamma.shape not in ((b,), (b, h)):
        raise ValueError(f"gla_decode_step: log_gamma must be [B] or [B, H], got "
                         f"{tuple(log_gamma.shape)}")
    if state.shape != (b, h, nf * nd + nf) or state.dtype != torch.float32 or \
            not state.is_contiguous():
        raise ValueError(f"gla_decode_step: state must be contiguous fp32 "
                         f"[B, H, F*D + F] = {(b, h, nf * nd + nf)}, got {tuple(state.shape)} "
                         f"{state.dtype}")
    _require_gpu(fq, fk, v, log_gamma, state)
    fq, fk, v = _bf16(fq), _bf16(fk), _bf16(v)
    lg = log_gamma.float().contiguous()
    y = torch.empty(b, h, nd, device=v.device, dtype=torch.bfloat16)
    rc = _lib.load().lz_gla_decode_step(_ptr(fq), _ptr(fk), _ptr(v), _ptr(lg), _ptr(state),
                                        _ptr(y), b, h, hk, nf, nd,
                                        int(lg.dim() == 2) | (GATE_LOGIT if gate_logit else 0),
                                        _stream(fq))
    _lib.check(rc, "lz_gla_decode_step")
    return y


def gla(fq, fk, v, log_gamma, chunk=CHUNK):
    """Chunked gated linear attention (``src/kernels/gla.py:259-263``).

    y_i = sum_{t<=i} w_it v_t / max(sum_{t<=i} w_it, FLT_MIN) with
    w_it = (fq_i . fk_t) exp(G_i - G_t), G = cumsum(log_gamma) along L.
    Returns bf16 ``[B, H, L, D]``.
    """
    _check_gla(fq, fk, v, log_gamma, chunk)
    if not (torch.is_grad_enabled() and (fq.requires_grad or fk.requires_grad or
                                         v.requires_grad or log_gamma.requires_grad)):
        # nothing to differentiate: the same forward launch without the
        # autograd node (and the same bits as with it)
        return _gla_fwd_launch(_bf16(fq), _bf16(fk), _bf16(v), _f32(log_gamma), False, chunk,
                               False)[0]
    return _GLA.apply(fq, fk, v, log_gamma, chunk)


# ---------------------------------------------------------------------------
# sliding-window softmax with sinks
# ---------------------------------------------------------------------------

def _check_swa(q, k, v, meta, window, fwd_blocks, bwd_blocks):
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"swa: q, k, v must be [B, H, L, d] of one shape, got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if meta.dim() != 1:
        raise ValueError(f"swa: meta must be 1-D, got {tuple(meta.shape)}")
    if not isinstance(window, int) or window < 1:
        raise ValueError(f"swa: window must be a positive int, got {window!r}")
    for blocks in (fwd_blocks, bwd_blocks):
        if blocks is FWD_BLOCKS or blocks is BWD_BLOCKS:   # the defaults, valid
            continue
        if len(tuple(blocks)) != 2 or any(int(x) < 1 for x in blocks):
            raise ValueError(f"swa: blocks must be two positive ints, got {blocks!r}")
    _require_gpu(q, k, v)
    if meta.numel():
        _require_gpu(meta)


def swa_forward(q, k, v, meta, window):
    """One ``lz_swa_fwd`` launch on bf16 contiguous q, k, v and fp32
    contiguous meta; returns (y, lse).  k and v may have fewer heads than q
    (a divisor, as in ``gla_forward``)."""
    _check_kv("swa_forward", q, k, v, q.shape[-1], q.shape[-1])
    return _swa_fwd_launch(q, k, v, meta, window)


def _swa_fwd_launch(q, k, v, meta, window):
    """``swa_forward`` without its shape checks (for callers that made them)."""
    b, h, length, d = q.shape
    y = torch.empty_like(q)
    lse = torch.empty(b, h, length, device=v.device, dtype=torch.float32)
    if y.numel():
        rc = _lib.load().lz_swa_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(meta), meta.numel(),
                                    _ptr(y), _ptr(lse), b, h, k.shape[1], length, d, window,
                                    1.0 / math.sqrt(d), _stream(q))
        _lib.check(rc, "lz_swa_fwd")
    return y, lse


def swa_backward(q, k, v, meta, lse, dy, window, grad_dtype):
    """One ``lz_swa_bwd`` launch: (dq, dk, dv) in grad_dtype, dmeta fp32;
    dk and dv per query head, also when k and v have fewer (kv) heads."""
    _check_kv("swa_backward", q, k, v, q.shape[-1], q.shape[-1])
    b, h, length, d = q.shape
    if tuple(dy.shape) != tuple(q.shape) or tuple(lse.shape) != (b, h, length):
        raise ValueError(f"swa_backward: dy must be {tuple(q.shape)} and lse {(b, h, length)}, "
                         f"got {tuple(dy.shape)} and {tuple(lse.shape)}")
    return _swa_bwd_launch(q, k, v, meta, lse, dy, window, grad_dtype)


def _swa_bwd_launch(q, k, v, meta, lse, dy, window, grad_dtype):
    """``swa_backward`` without its shape checks (for callers that made them)."""
    b, h, length, d = q.shape
    dq = torch.empty(q.shape, device=q.device, dtype=grad_dtype)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    dmeta = torch.empty(meta.shape, device=q.device, dtype=torch.float32)
    if dy.numel():
        lib = _lib.load()
        n_meta = meta.numel()
        nbytes = _swa_bwd_ws(b, h, length, d, n_meta)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        rc = lib.lz_swa_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(meta), n_meta,
                            _ptr(lse), _ptr(dy), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dmeta),
                            int(grad_dtype == torch.bfloat16), b, h, k.shape[1], length, d, window,
                            1.0 / math.sqrt(d), _ptr(ws), ws.numel(), _stream(q))
        _lib.check(rc, "lz_swa_bwd")
    else:
        dq.zero_(), dk.zero_(), dv.zero_(), dmeta.zero_()
    return dq, dk, dv, dmeta


SWA_DECODE_MAX_WINDOW = 8192


def swa_decode_step(q, k_cache, v_cache, meta, pos):
    """The ``swa`` output row of one new query per (b, h) at absolute
    position ``pos`` (src/kernels/swa.py:19-59 at i = pos), against a
    ring-buffered window cache.  The reference has no decode path.

    q ``[B, H, d]`` (RoPE applied), k_cache / v_cache ``[B, Hkv, W, d]``
    holding position p in slot p % W (the caller has written position pos
    there), meta ``[n_meta]`` fp32.  Returns bf16 ``[B, H, d]``; no autograd."""
    if q.dim() != 3 or k_cache.dim() != 4 or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError(f"swa_decode_step: q [B, H, d] and k_cache, v_cache [B, Hkv, W, d] "
                         f"expected, got {tuple(q.shape)}, {tuple(k_cache.shape)}, "
                         f"{tuple(v_cache.shape)}")
    b, h, d = q.shape
    hk, window = k_cache.shape[1], k_cache.shape[2]
    if k_cache.shape[0] != b or k_cache.shape[3] != d or hk <= 0 or h % hk:
        raise ValueError(f"swa_decode_step: caches must be [B, Hkv, W, d] = [{b}, Hkv, W, {d}] "
                         f"with Hkv dividing {h}, got {tuple(k_cache.shape)}")
    if not 1 <= window <= SWA_DECODE_MAX_WINDOW:
        raise ValueError(f"swa_decode_step: window must be in [1, {SWA_DECODE_MAX_WINDOW}], "
                         f"got {window}")
    if not isinstance(pos, int) or pos < 0:
        raise ValueError(f"swa_decode_step: pos must be a non-negative int, got {pos!r}")
    if meta.dim() != 1:
        raise ValueError(f"swa_decode_step: meta must be 1-D, got {tuple(meta.shape)}")
    _require_gpu(q, k_cache, v_cache)
    q, kc, vc, meta = _bf16(q), _bf16(k_cache), _bf16(v_cache), _f32(meta)
    y = torch.empty_like(q)
    if y.numel():
        rc = _lib.load().lz_swa_decode_step(_ptr(q), _ptr(kc), _ptr(vc), _ptr(meta),
                                            meta.numel(), _ptr(y), b, h, hk, window, d, pos,
                                            1.0 / math.sqrt(d), _stream(q))
        _lib.check(rc, "lz_swa_decode_step")
    return y


class _SWA(torch.autograd.Function):
    """Autograd node of ``swa``; mirrors ``_SWA`` (src/kernels/swa.py:136-179)."""

    @staticmethod
    def forward(ctx, q, k, v, meta, window, fwd_blocks, bwd_blocks):
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, meta.dtype)
        q, k, v = _bf16(q), _bf16(k), _bf16(v)
        meta = _f32(meta)
        y, lse = _swa_fwd_launch(q, k, v, meta, window)
        if any(ctx.needs_input_grad[:4]):
            ctx.save_for_backward(q, k, v, meta, lse)
        ctx.window = window
        return y

    @staticmethod
    def backward(ctx, dy):
        q, k, v, meta, lse = ctx.saved_tensors
        gdt = torch.bfloat16 if all(x == torch.bfloat16 for x in ctx.dtypes[:3]) else torch.float32
        grads = _swa_bwd_launch(q, k, v, meta, lse, _bf16(dy), ctx.window, gdt)
        return _cast_grads(grads, ctx.dtypes) + (None, None, None)


def swa(q, k, v, meta, window, fwd_blocks=FWD_BLOCKS, bwd_blocks=BWD_BLOCKS):
    """Sliding-window softmax attention with sink logits (``src/kernels/swa.py:182-183``).

    y_i = sum_{i-W<t<=i} e^{s_it} v_t / (sum_j e^{meta_j} + sum_t e^{s_it}),
    s_it = q_i . k_t / sqrt(d).  Returns bf16 ``[B, H, L, d]``.
    """
    _check_swa(q, k, v, meta, window, fwd_blocks, bwd_blocks)
    if not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or
                                         v.requires_grad or meta.requires_grad)):
        # nothing to differentiate: the forward launch without the autograd node
        return _swa_fwd_launch(_bf16(q), _bf16(k), _bf16(v), _f32(meta), window)[0]
    return _SWA.apply(q, k, v, meta, window, tuple(fwd_blocks), tuple(bwd_blocks))
