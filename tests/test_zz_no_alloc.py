"""lz_gla_fwd_noalloc (the GLA forward whose segment states live in the
library's static device array instead of a caller workspace) against
lz_gla_fwd with a workspace, through the C ABI, on two calls in a row -- the
second smaller -- plus the oracle on the second."""
import pytest
import torch

from lizard_reproduction_amd import _lib
from oracle import lizard_oracle as lo
from tests.helpers import OUT_TOL, baseline_gla_inputs, max_rel

pytestmark = pytest.mark.gpu


def _run(lib, fq, fk, v, lg, noalloc):
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    per_head = int(lg.dim() == 3)
    y = torch.empty(b, h, length, nd, device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    args = (fq.data_ptr(), fk.data_ptr(), v.data_ptr(), lg.data_ptr(), y.data_ptr(), b, h, h,
            length, nf, nd, per_head, 64)
    if noalloc:
        rc = lib.lz_gla_fwd_noalloc(*args, stream)
        _lib.check(rc, "lz_gla_fwd_noalloc")
    else:
        nbytes = lib.lz_gla_fwd_workspace_bytes(b, h, length, nf, nd, per_head, 64)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        rc = lib.lz_gla_fwd(*args, ws.data_ptr(), nbytes, stream)
        _lib.check(rc, "lz_gla_fwd")
    torch.cuda.synchronize()
    return y


def test_init_then_noalloc_forward():
    """lz_init (the no-allocation forward's per-device set-up, made outside a
    capture by callers that capture) succeeds, again when repeated, and the
    forward after it matches the workspace forward."""
    lib = _lib.load()
    assert lib.lz_init() == 0, lib.lz_last_error()
    assert lib.lz_init() == 0, lib.lz_last_error()
    fq, fk, v, lg, _ = baseline_gla_inputs(1, 8, 700, 64, True, 2.0, 1.5, seed=5)
    dev = [t.cuda().contiguous() for t in (fq, fk, v, lg)]
    assert torch.equal(_run(lib, *dev, noalloc=True), _run(lib, *dev, noalloc=False))


@pytest.mark.parametrize("order", ["noalloc_first", "workspace_first"])
def test_noalloc_forward_equals_workspace_forward(order):
    lib = _lib.load()
    # call 1: B*H = 32 at F = D = 128 -> 16 segments per (b, h), 32 MiB of
    # states; call 2: a smaller input (B*H = 4, F = D = 64, 1000 tokens,
    # one gate per token) -> 16 one-chunk segments, written over call 1's
    cases = [(1, 32, 4096, 128, True, 2.0, 1.5), (1, 4, 1000, 64, False, 3.0, 1.0)]
    for i, (b, h, length, d, per_head, mean, std) in enumerate(cases):
        print(f"[noalloc] call {i + 1}: B={b} H={h} L={length} F=D={d} per_head={per_head}",
              flush=True)
        fq, fk, v, lg, _ = baseline_gla_inputs(b, h, length, d, per_head, mean, std, seed=i)
        assert lib.lz_gla_fwd_workspace_bytes(b, h, length, d, d, int(per_head), 64) > 0
        dev = [t.cuda().contiguous() for t in (fq, fk, v, lg)]
        if order == "noalloc_first":
            ours = _run(lib, *dev, noalloc=True)
            ref = _run(lib, *dev, noalloc=False)
        else:
            ref = _run(lib, *dev, noalloc=False)
            ours = _run(lib, *dev, noalloc=True)
        # the same kernels on the same split: bitwise the same output
        assert torch.equal(ours, ref), (i, max_rel(ours, ref))
        if i == 1:
            expected = lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float32)
            err = max_rel(ours, expected)
            print(f"[noalloc] call 2 vs oracle: {err:.2e}", flush=True)
            assert err <= OUT_TOL


def test_noalloc_forward_without_segments_and_bad_arguments():
    """B*H = 512 fills the GPU without segments (no scratch used); bad
    arguments are refused before any launch, as by lz_gla_fwd."""
    lib = _lib.load()
    fq, fk, v, lg, _ = baseline_gla_inputs(16, 32, 256, 64, True, 2.0, 1.5)
    assert lib.lz_gla_fwd_workspace_bytes(16, 32, 256, 64, 64, 1, 64) == 0
    dev = [t.cuda().contiguous() for t in (fq, fk, v, lg)]
    assert torch.equal(_run(lib, *dev, noalloc=True), _run(lib, *dev, noalloc=False))
    p = dev[0].data_ptr()
    rc = lib.lz_gla_fwd_noalloc(p, p, p, p, None, 1, 1, 1, 8, 16, 16, 0, 64, None)
    assert rc != 0 and b"null" in lib.lz_last_error()
    rc = lib.lz_gla_fwd_noalloc(p, p, p, p, p, 1, 1, 1, 8, 300, 16, 0, 64, None)
    assert rc != 0 and b"unsupported" in lib.lz_last_error()
