"""Parity at BASELINE.json's full sizes.  The dense oracle cannot hold these
(L x L per (b, h)), so the HIP kernels run on the whole batch and sampled
(b, h) slices are checked against the chunked fp64 restatement
(oracle.gla_chunked, pinned against the dense oracle in tests/test_oracle.py)
with autograd for the gradients; plus size-independent properties over the
whole output (constant values stay constant, bitwise determinism)."""
import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import GRAD_TOL, OUT_TOL, baseline_gla_inputs, max_rel

pytestmark = pytest.mark.gpu


def check_slices(batch, heads, length, dim, per_head, mean, std, slices, label):
    fq, fk, v, lg, dy = baseline_gla_inputs(batch, heads, length, dim, per_head, mean, std)
    ours = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
    y = kernels.gla(*ours)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    worst = {}
    for b, h in slices:
        sl = [t[b:b + 1, h:h + 1].double().requires_grad_() for t in (fq, fk, v)]
        g = (lg[b:b + 1, h:h + 1] if per_head else lg[b:b + 1]).double().requires_grad_()
        ref = lo.gla_chunked(*sl, g, 64)
        ref.backward(dy[b:b + 1, h:h + 1].double())
        pairs = {"y": (y[b, h], ref[0, 0]), "dfq": (ours[0].grad[b, h], sl[0].grad[0, 0]),
                 "dfk": (ours[1].grad[b, h], sl[1].grad[0, 0]),
                 "dv": (ours[2].grad[b, h], sl[2].grad[0, 0])}
        if per_head:
            pairs["dlg"] = (ours[3].grad[b, h], g.grad[0, 0])
        for k, (a, r) in pairs.items():
            worst[k] = max(worst.get(k, 0.0), max_rel(a, r))
    print(f"[parity] {label} slices {slices}: " +
          " ".join(f"{k}={v:.2e}" for k, v in worst.items()), flush=True)
    assert worst["y"] <= OUT_TOL, worst
    for k, e in worst.items():
        if k != "y":
            assert e <= GRAD_TOL, (k, worst)


def test_headline_shape_slices_match_chunked_oracle():
    """B=16, H=32, L=2048, F=D=128, per-head gate (the north-star forward
    shape), forward and backward."""
    check_slices(16, 32, 2048, 128, True, 2.0, 1.5, [(0, 0), (7, 13), (15, 31)], "headline")


def test_config4_longest_slices_match_chunked_oracle():
    """B=16, H=32, L=16384, F=D=128, per-head gate (the largest config-4
    point), forward and backward."""
    check_slices(16, 32, 16384, 128, True, 2.0, 1.5, [(3, 5), (12, 30)], "config4 L=16K")


@pytest.mark.parametrize("batch, length, slices", [
    (1, 4096, [(0, 0), (0, 17), (0, 31)]),      # 16 segments of 4 chunks
    (1, 16384, [(0, 5), (0, 30)]),              # 16 segments of 16 chunks
    (4, 2048, [(0, 0), (2, 9), (3, 31)]),       # 4 segments of 8 chunks (records folded)
    (4, 8192, [(1, 3), (3, 28)])])              # 4 segments of 32 chunks (records folded)
def test_config4_segmented_d128_walks_slices_match_chunked_oracle(batch, length, slices):
    """The config-4 sweep points whose B*H (32, 128) cannot fill the GPU:
    each (b, h) sequence is cut into segments of several chunks, so the
    F=D=128 segment state passes run, then either the forward and reverse
    segment scans and walks that start from a scanned state (16 segments)
    or walks that fold the records themselves (4 segments); output and
    every gradient (d log_gamma per head) of sampled slices against the
    chunked fp64 oracle."""
    from lizard_reproduction_amd import _lib
    lib = _lib.load()
    assert lib.lz_gla_fwd_workspace_bytes(batch, 32, length, 128, 128, 1, 64) > 0  # segmented
    check_slices(batch, 32, length, 128, True, 2.0, 1.5, slices,
                 f"config4 segmented B={batch} L={length}")


def test_reverse_order_state_pass_with_a_shared_gate_matches_chunked_oracle():
    """B=1 L=16384 F=D=128 with one gate per token (config 2's gate on the
    config-4 shape): the forward state pass walks its segments from the last
    chunk (251 MB of fk and v rows), scanning the shared gate row backwards;
    output and gradients of sampled slices against the chunked fp64 oracle."""
    check_slices(1, 32, 16384, 128, False, 3.0, 1.0, [(0, 2), (0, 27)],
                 "config4 shape, per-token gate, B=1 L=16384")


@pytest.mark.parametrize("batch, length", [(1, 16384), (4, 8192)])
def test_reverse_order_state_pass_gives_the_backward_the_same_records(batch, length):
    """At these shapes the forward state pass reads more than 128 MB of fk
    and v (251 and 403 MB), so it walks each segment from its last chunk to
    its first.  The backward given the forward's records and the backward
    that recomputes them must agree bit for bit; the slices above check the
    same shapes against the oracle."""
    fq, fk, v, lg, dy = baseline_gla_inputs(batch, 32, length, 128, True, 2.0, 1.5)
    fq, fk, v, lg, dy = (t.cuda() for t in (fq, fk, v, lg, dy))
    _, state = kernels.gla_forward(fq, fk, v, lg, keep_state=True)
    assert state is not None   # segmented
    kept = kernels.gla_backward(fq, fk, v, lg, dy, state, torch.bfloat16)
    again = kernels.gla_backward(fq, fk, v, lg, dy, None, torch.bfloat16)
    for name, a, b in zip(("dfq", "dfk", "dv", "dlog_gamma"), kept, again):
        assert torch.equal(a, b), name


def test_headline_shape_constant_values_stay_constant_everywhere():
    """y_i is a normalised average of v, so a constant v comes back (up to
    the bf16 rounding of the state operand) at every position of every
    (b, h) -- a check over the whole output, not a sample."""
    fq, fk, _, lg, _ = baseline_gla_inputs(16, 32, 2048, 128, True, 2.0, 1.5)
    v = torch.full((16, 32, 2048, 128), 0.37, dtype=torch.bfloat16)
    with torch.no_grad():
        y = kernels.gla(fq.cuda(), fk.cuda(), v.cuda(), lg.cuda())
    err = ((y.float() - 0.37).abs().max() / 0.37).item()
    print(f"[parity] headline constant v: max rel {err:.2e}", flush=True)
    assert err <= OUT_TOL


def test_headline_shape_is_deterministic():
    fq, fk, v, lg, dy = baseline_gla_inputs(16, 32, 2048, 128, True, 2.0, 1.5)
    runs = []
    for _ in range(2):
        leaves = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
        y = kernels.gla(*leaves)
        y.backward(dy.cuda())
        runs.append([y.detach()] + [t.grad for t in leaves])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_headline_shape_every_row_matches_per_row_calls():
    """At the headline shape each backward walk launches twice as many
    workgroups as there are CUs, so it runs in two rounds, and the dkv walk
    takes its blocks in reverse launch order per XCD.  Every (b, h) of the
    output and of every gradient is compared with the same call made one
    batch row at a time (32 (b, h) per call: segmented walks in one round,
    whose parity the segmented tests above pin), so a block that the order
    skipped or computed twice fails somewhere in the whole tensors."""
    fq, fk, v, lg, dy = baseline_gla_inputs(16, 32, 2048, 128, True, 2.0, 1.5)
    leaves = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
    y = kernels.gla(*leaves)
    y.backward(dy.cuda())
    worst = {}
    for b in range(16):
        row = [t[b:b + 1].cuda().requires_grad_() for t in (fq, fk, v, lg)]
        yr = kernels.gla(*row)
        yr.backward(dy[b:b + 1].cuda())
        pairs = {"y": (y[b], yr[0])}
        for name, full, part in zip(("dfq", "dfk", "dv", "dlg"), leaves, row):
            pairs[name] = (full.grad[b], part.grad[0])
        for k, (a, r) in pairs.items():
            worst[k] = max(worst.get(k, 0.0), max_rel(a, r))
    print("[parity] headline whole batch vs per-row calls: " +
          " ".join(f"{k}={e:.2e}" for k, e in worst.items()), flush=True)
    assert worst["y"] <= OUT_TOL, worst
    for k, e in worst.items():
        if k != "y":
            assert e <= GRAD_TOL, (k, worst)


def config5_attention_inputs():
    """The layer's GLA call at BASELINE config 5: B=4, H=32, L=4096, F=256
    (Hedgehog maps [softmax(x), softmax(-x)] of 128 features), D=64, one gate
    per token (logsigmoid(N(3, 1))), dO ~ N(0, 1); forward and backward of
    the whole batch on the GPU.  Returns the CPU inputs, dO, y and the leaves."""
    g = torch.Generator().manual_seed(9)
    b, h, length = 4, 32, 4096

    def hedgehog(x):
        return torch.cat([x.softmax(-1), (-x).softmax(-1)], -1).bfloat16()
    fq = hedgehog(torch.randn(b, h, length, 128, generator=g))
    fk = hedgehog(torch.randn(b, h, length, 128, generator=g))
    v = torch.randn(b, h, length, 64, generator=g).bfloat16()
    lg = F.logsigmoid(3 + torch.randn(b, length, generator=g))
    dy = torch.randn(b, h, length, 64, generator=g).bfloat16()
    ours = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
    y = kernels.gla(*ours)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    return (fq, fk, v, lg), dy, y, ours


def test_config5_attention_shape_slices_match_chunked_oracle():
    """Sampled (b, h) slices of the config-5 attention call against the
    chunked fp64 oracle: output, dfq, dfk, dv."""
    (fq, fk, v, lg), dy, y, ours = config5_attention_inputs()
    worst = {}
    for bi, hi in [(0, 0), (2, 17), (3, 31)]:
        sl = [t[bi:bi + 1, hi:hi + 1].double().requires_grad_() for t in (fq, fk, v)]
        gl = lg[bi:bi + 1].double().requires_grad_()
        ref = lo.gla_chunked(*sl, gl, 64)
        ref.backward(dy[bi:bi + 1, hi:hi + 1].double())
        pairs = {"y": (y[bi, hi], ref[0, 0]), "dfq": (ours[0].grad[bi, hi], sl[0].grad[0, 0]),
                 "dfk": (ours[1].grad[bi, hi], sl[1].grad[0, 0]),
                 "dv": (ours[2].grad[bi, hi], sl[2].grad[0, 0])}
        for k, (a, r) in pairs.items():
            worst[k] = max(worst.get(k, 0.0), max_rel(a, r))
    print("[parity] config5 attention slices: " +
          " ".join(f"{k}={v:.2e}" for k, v in worst.items()), flush=True)
    assert worst["y"] <= OUT_TOL, worst
    for k, e in worst.items():
        if k != "y":
            assert e <= GRAD_TOL, (k, worst)


def test_config5_attention_shape_shared_gate_gradient_matches_chunked_oracle():
    """One whole batch row (all 32 heads) of the config-5 attention call
    against the chunked fp64 oracle, so that the gradient of the gate shared
    by the heads -- summed over the heads and reverse-cumsummed over the 4096
    tokens inside the kernels -- is compared too, with the output and the
    other gradients of every head of the row."""
    (fq, fk, v, lg), dy, y, ours = config5_attention_inputs()
    bi = 2
    sl = [t[bi:bi + 1].double().requires_grad_() for t in (fq, fk, v)]
    gl = lg[bi:bi + 1].double().requires_grad_()
    ref = lo.gla_chunked(*sl, gl, 64)
    ref.backward(dy[bi:bi + 1].double())
    errs = {"y": max_rel(y[bi], ref[0]), "dfq": max_rel(ours[0].grad[bi], sl[0].grad[0]),
            "dfk": max_rel(ours[1].grad[bi], sl[1].grad[0]),
            "dv": max_rel(ours[2].grad[bi], sl[2].grad[0]),
            "dlg": max_rel(ours[3].grad[bi], gl.grad[0])}
    print("[parity] config5 attention row 2, all heads: " +
          " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["y"] <= OUT_TOL, errs
    for k, e in errs.items():
        if k != "y":
            assert e <= GRAD_TOL, (k, errs)
