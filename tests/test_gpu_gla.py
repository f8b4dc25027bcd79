"""GPU parity of the HIP GLA path against the CPU oracle.

Mirrors the reference's kernel tests (tests/test_kernels.py:55-107): same
inputs, lengths, chunk sizes, per-head gates, strong decay and the
no-grad/grad bitwise check, with the north-star bar (max-abs error relative
to the fp32 oracle's max-abs: <= 1e-2 outputs, <= 2e-2 gradients) on top of
the reference's own norm bar.  The BASELINE shapes are checked against the
dense oracle where it fits and against the chunked oracle beyond.
"""
import pytest
import torch
import torch.nn.functional as F

from lizard_reproduction_amd import kernels
from oracle import lizard_oracle as lo
from tests.helpers import (GRAD_TOL, OUT_TOL, baseline_gla_inputs, compare, gla_inputs,
                           max_rel)

pytestmark = pytest.mark.gpu


def gla_kernel(chunk):
    def kernel(fq, fk, v, z):
        return kernels.gla(fq, fk, v, F.logsigmoid(z), chunk)
    return kernel


def gla_reference(fq, fk, v, z):
    return lo.gla_kernel_api(fq, fk, v, F.logsigmoid(z), dtype=torch.float32)


@pytest.mark.parametrize("length, chunk", [(1, 16), (77, 16), (150, 64), (64, 64), (129, 64)])
def test_gla_matches_oracle(length, chunk):
    inputs = gla_inputs(length)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(chunk), gla_reference, inputs, grad, label=f"L={length}")


def test_gla_with_a_gate_per_head_matches_oracle():
    inputs = gla_inputs(100, gates=(3,))
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(16), gla_reference, inputs, grad, label="per-head")


def test_gla_with_strong_decay_matches_oracle():
    inputs = gla_inputs(200, shift=-6.0)
    assert F.logsigmoid(inputs[3]).sum(-1).max() < -1000
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(16), gla_reference, inputs, grad, label="strong decay")


@pytest.mark.parametrize("features, dim", [(64, 64), (128, 128), (256, 64), (32, 128), (128, 32),
                                           (40, 72), (256, 32), (232, 64), (256, 40)])
def test_gla_feature_and_value_dims(features, dim):
    inputs = gla_inputs(150, batch=1, heads=2, features=features, dim=dim)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad, label=f"F={features} D={dim}")


def test_gla_without_grad_gives_the_same_output():
    fq, fk, v, z = (t.cuda() for t in gla_inputs(70))
    y = kernels.gla(fq, fk, v.requires_grad_(), F.logsigmoid(z), 16)
    with torch.no_grad():
        assert torch.equal(kernels.gla(fq, fk, v, F.logsigmoid(z), 16), y)


@pytest.mark.parametrize("gates", [(), (32,)])
def test_gla_no_grad_walk_with_nontemporal_loads_gives_the_same_output(gates):
    """Enough (b, h) to fill the GPU without segments (no forward workspace):
    there the no-grad forward passes the no-reuse hint and its walk loads the
    chunks nontemporally, while a forward kept for a backward loads them
    normally.  The cache policy must not change a bit of y."""
    from lizard_reproduction_amd import _lib
    assert _lib.load().lz_gla_fwd_workspace_bytes(16, 32, 200, 128, 128, len(gates), 64) == 0
    fq, fk, v, z = (t.cuda() for t in gla_inputs(200, gates=gates, batch=16, heads=32,
                                                 features=128, dim=128))
    y = kernels.gla(fq, fk, v.requires_grad_(), F.logsigmoid(z))
    with torch.no_grad():
        assert torch.equal(kernels.gla(fq, fk, v, F.logsigmoid(z)), y)


def test_gla_is_deterministic():
    fq, fk, v, z = (t.cuda().requires_grad_() for t in gla_inputs(150, gates=(3,)))
    outs = []
    for _ in range(2):
        y = kernels.gla(fq, fk, v, F.logsigmoid(z))
        y.backward(torch.ones_like(y))
        outs.append([y.detach().clone()] + [t.grad.clone() for t in (fq, fk, v, z)])
        for t in (fq, fk, v, z):
            t.grad = None
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_gla_fp32_inputs_give_fp32_grads():
    fq, fk, v, z = gla_inputs(50)
    leaves = [t.float().cuda().requires_grad_() for t in (fq, fk, v)]
    lg = F.logsigmoid(z).cuda().requires_grad_()
    y = kernels.gla(*leaves, lg)
    y.float().sum().backward()
    assert y.dtype == torch.bfloat16
    assert all(t.grad.dtype == torch.float32 for t in leaves + [lg])


@pytest.mark.parametrize("gates", [(64,), ()])
def test_gla_one_segment_fp32_grads_match_oracle(gates):
    # B*H = 512 fills the GPU without segments: the dq and dkv walks of each
    # (b, h) run in one workgroup, here writing fp32 gradients (fp32 inputs)
    inputs = gla_inputs(100, gates=gates, batch=8, heads=64, features=32, dim=32, seed=23)
    inputs = [t.float() if t.dtype == torch.bfloat16 else t for t in inputs]
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(5))
    from lizard_reproduction_amd import _lib
    assert _lib.load().lz_gla_fwd_workspace_bytes(8, 64, 100, 32, 32, len(gates), 64) == 0
    compare(gla_kernel(64), lambda *a: lo.gla_chunked(*a[:3], F.logsigmoid(a[3]), chunk=64,
                                                      dtype=torch.float32),
            inputs, grad, label=f"one segment fp32 grads gates={gates}")


def _baseline_case(batch, heads, length, dim, per_head, gate_mean, gate_std, oracle):
    fq, fk, v, lg, dy = baseline_gla_inputs(batch, heads, length, dim, per_head,
                                            gate_mean, gate_std)
    ours = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
    y = kernels.gla(*ours)
    y.backward(dy.cuda())
    theirs = [t.clone().requires_grad_() for t in (fq, fk, v, lg)]
    ref = oracle(*theirs)
    ref.backward(dy.float())
    errs = [max_rel(y, ref)] + [max_rel(a.grad, b.grad) for a, b in zip(ours, theirs)]
    print(f"GLA B={batch} H={heads} L={length} d={dim} per_head={per_head}: "
          f"out {errs[0]:.2e} grads " + " ".join(f"{e:.2e}" for e in errs[1:]), flush=True)
    assert errs[0] <= OUT_TOL, errs
    assert max(errs[1:]) <= GRAD_TOL, errs


def test_gla_baseline_config1_dense():
    _baseline_case(1, 4, 256, 64, False, 3.0, 1.0,
                   lambda *a: lo.gla_kernel_api(*a, dtype=torch.float32))


def test_gla_baseline_config2_training_shape_dense():
    _baseline_case(1, 32, 2048, 64, False, 3.0, 1.0,
                   lambda *a: lo.gla_kernel_api(*a, dtype=torch.float32))


def test_gla_baseline_config4_per_head_d128_chunked():
    # B=1, L=2048 of the config-4 sweep; oracle = chunked restatement in fp32
    # (pinned against the dense oracle in tests/test_oracle.py)
    _baseline_case(1, 4, 2048, 128, True, 2.0, 1.5,
                   lambda *a: lo.gla_chunked(*a, chunk=64, dtype=torch.float32))


@pytest.mark.parametrize("batch, heads, length", [(8, 64, 200), (1, 512, 333)])
def test_gla_single_segment_walk(batch, heads, length):
    # B*H >= 512 fills the GPU with one workgroup per (b, h): every workgroup
    # walks all chunks of its sequence (no segment split)
    inputs = gla_inputs(length, batch=batch, heads=heads, features=32, dim=32)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad, label=f"B*H={batch * heads} L={length}")


@pytest.mark.parametrize("length", [64 * 24, 64 * 24 + 17])
def test_gla_segments_of_several_chunks(length):
    # B*H = 64: the sequence is split into 8 (or 7) segments of 3 (or 4)
    # chunks, whose entering states come from the segment pass and scan
    inputs = gla_inputs(length, batch=4, heads=16, features=64, dim=64)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad, label=f"segments L={length}")


@pytest.mark.parametrize("features", [150, 200])
def test_gla_state_pass_feature_slices_with_ragged_features(features):
    # B*H = 2 and F in (128, 256]: the segment state pass splits the record's
    # 256 feature rows over 4 workgroups of 64; at F = 150 the third slice
    # holds 22 columns of fk and the fourth none (its record rows stay zero)
    inputs = gla_inputs(700, batch=1, heads=2, features=features, dim=64, seed=9)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad, label=f"sliced state pass F={features}")


@pytest.mark.parametrize("batch, heads, length, dim, per_head", [
    (1, 2, 64 * 11 + 5, 64, True), (2, 3, 64 * 9, 32, False), (1, 1, 1, 64, False)])
def test_gla_wide_features_segments(batch, heads, length, dim, per_head):
    # F = 256 (the eight-wave walk): small B*H, so the sequence is split into
    # segments and each walk workgroup takes two of them
    inputs = gla_inputs(length, gates=(heads,) if per_head else (), batch=batch, heads=heads,
                        features=256, dim=dim, seed=5)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad,
            label=f"F=256 D={dim} B*H={batch * heads} L={length}")


@pytest.mark.parametrize("batch, heads, length, features, dim, per_head", [
    (2, 64, 64 * 7 + 13, 128, 128, False),   # B*H = 128: 4 segments of 2 chunks
    (4, 50, 300, 128, 64, True),              # B*H = 200: 3 segments, the last short
    (1, 128, 200, 64, 128, False),            # 4 one-chunk segments, the last ragged
    (2, 64, 500, 256, 64, False),             # eight-wave walks, two segments each
])
def test_gla_walks_fold_few_segments(batch, heads, length, features, dim, per_head):
    # at most 4 segments per (b, h) with records of at least 128 x 64 floats:
    # the walks fold the segment records themselves (no scan launch), in the
    # forward, the dq walk (left to right) and the dkv walk (right to left)
    inputs = gla_inputs(length, gates=(heads,) if per_head else (), batch=batch, heads=heads,
                        features=features, dim=dim, seed=13)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(2))
    compare(gla_kernel(64), lambda *a: lo.gla_chunked(*a[:3], F.logsigmoid(a[3]), chunk=64,
                                                      dtype=torch.float32),
            inputs, grad, label=f"folded segments F={features} D={dim} B*H={batch * heads}")


def test_gla_segmented_dkv_walk_in_rounds_matches_oracle():
    # B*H = 100 with 10 chunks: 5 segments of 2 chunks per (b, h) and 500
    # dkv-walk workgroups at one per CU, so that walk runs in rounds and takes
    # its blocks in reverse launch order per XCD
    inputs = gla_inputs(600, gates=(50,), batch=2, heads=50, features=64, dim=64, seed=17)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(4))
    compare(gla_kernel(64), lambda *a: lo.gla_chunked(*a[:3], F.logsigmoid(a[3]), chunk=64,
                                                      dtype=torch.float32),
            inputs, grad, label="dkv walk in rounds B*H=100 L=600")


def test_gla_backward_without_forward_workspace_is_bitwise_equal():
    # through the C ABI: lz_gla_bwd given no forward workspace recomputes the
    # state entering each segment; the gradients must be the same bits as the
    # autograd path, which hands it the forward's workspace
    from lizard_reproduction_amd import _lib
    fq, fk, v, z = gla_inputs(700, batch=1, heads=4, features=64, dim=64)
    lg = F.logsigmoid(z)
    leaves = [t.cuda().requires_grad_() for t in (fq, fk, v, lg)]
    y = kernels.gla(*leaves)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(3)).bfloat16().cuda()
    y.backward(dy)
    lib = _lib.load()
    b, h, length, nf = fq.shape
    nd = v.shape[-1]
    assert lib.lz_gla_fwd_workspace_bytes(b, h, length, nf, nd, 0, 64) > 0   # segmented
    ins = [t.detach().contiguous() for t in leaves]
    dfq, dfk, dv = (torch.empty_like(t) for t in ins[:3])
    dlg = torch.empty_like(ins[3])
    n = lib.lz_gla_bwd_workspace_bytes(b, h, length, nf, nd, 0, 64)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    rc = lib.lz_gla_bwd(*(t.data_ptr() for t in ins), dy.data_ptr(), dfq.data_ptr(),
                        dfk.data_ptr(), dv.data_ptr(), dlg.data_ptr(), 1, b, h, h, length, nf,
                        nd, 0, 64, None, 0, ws.data_ptr(), n,
                        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "lz_gla_bwd")
    torch.cuda.synchronize()
    for ours, ref in zip((dfq, dfk, dv, dlg), leaves):
        assert torch.equal(ours, ref.grad)


@pytest.mark.parametrize("features, dim, length, heads, gates", [
    (256, 128, 150, 2, ()),      # head_dim-128 models at feature_dim 128: two D tiles of 64
    (512, 64, 150, 2, ()),       # feature_dim 256: two F tiles, numerators summed
    (300, 200, 130, 2, (2,)),    # ragged F and D tiles together, per-head gate
    (24, 300, 77, 2, ()),        # D tiles of a small F
    (512, 64, 1000, 3, (3,)),    # segmented walks inside each F tile (16 one-chunk segments)
    (1024, 128, 200, 1, ()),     # eight F tiles of 128, one D tile
])
def test_gla_sizes_past_the_walks_match_oracle(features, dim, length, heads, gates):
    """The reference's kernels take any F and D (src/kernels/gla.py:74,154,171,
    203-210); past the walks' own sizes the library runs them on tiles."""
    inputs = gla_inputs(length, gates=gates, batch=1, heads=heads, features=features, dim=dim)
    assert not kernels.gla_native(features, dim)
    grad = torch.randn(inputs[2].shape, generator=torch.Generator().manual_seed(1))
    compare(gla_kernel(64), gla_reference, inputs, grad,
            label=f"tiled F={features} D={dim} L={length}")


def test_gla_tiled_sizes_fp32_grads_determinism_and_no_grad_equality():
    fq, fk, v, z = gla_inputs(90, batch=1, heads=2, features=512, dim=64)
    leaves = [t.float().cuda().requires_grad_() for t in (fq, fk, v)]
    lg = F.logsigmoid(z).cuda().requires_grad_()
    outs = []
    for _ in range(2):
        y = kernels.gla(*leaves, lg)
        y.float().sum().backward()
        outs.append([y.detach().clone()] + [t.grad.clone() for t in leaves + [lg]])
        for t in leaves + [lg]:
            t.grad = None
    assert all(g.dtype == torch.float32 for g in outs[0][1:])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    with torch.no_grad():
        assert torch.equal(kernels.gla(*[t.detach() for t in leaves], lg.detach()), outs[0][0])


def test_gla_tiled_constant_values_stay_constant():
    """y is a normalised average of v also when the numerator and the
    denominator are sums over F tiles (each tile's bf16 weights feed both)."""
    fq, fk, _, z = gla_inputs(300, batch=1, heads=2, features=600, dim=96)
    v = torch.full((1, 2, 300, 96), -1.25, dtype=torch.bfloat16)
    with torch.no_grad():
        y = kernels.gla(fq.cuda(), fk.cuda(), v.cuda(), F.logsigmoid(z).cuda())
    assert ((y.float() + 1.25).abs().max() / 1.25).item() <= OUT_TOL
