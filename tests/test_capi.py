"""CPU tests of the boundary: the C-ABI library builds, loads, exports every
symbol include/lizard_hip.h declares, rejects bad arguments with a message
(without touching a GPU), and the product never reaches the oracle.

The bad-argument tests pass null or dummy device pointers (``c_void_p(16)``)
and expect the library's own checks to refuse the call.  They run only where
no GPU is visible (``no_gpu`` below): there a call that the checks let through
fails at its launch for want of a device, which ``refused`` reports as a
failure, while on a machine with a GPU the same call would launch kernels on
those addresses."""
import ctypes
import os
import re

import pytest
import torch

from lizard_reproduction_amd import _lib, kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lizard_hip.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from lizard_reproduction_amd import build
        build.build(verbose=False)
    return _lib.load()


# Tests that hand the library null or dummy device pointers: CPU machines only.
no_gpu = pytest.mark.skipif(
    torch.cuda.is_available(),
    reason="passes dummy device pointers; a call the checks missed would launch on them")


def refused(lib, rc, needle=None):
    """A bad-argument call was refused by the library's own checks: a nonzero
    code and a validation message, never a HIP error.  These calls pass dummy
    pointers, so one that got past the checks would reach a kernel launch
    (here it fails for want of a device; on a machine with a GPU it would
    read and write those addresses)."""
    msg = lib.lz_last_error()
    assert rc != 0, msg
    assert b"HIP error" not in msg, msg
    if needle is not None:
        assert needle in msg, msg


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(lz_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(raw, name), name


def test_abi_version_and_error_string(lib):
    assert lib.lz_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.lz_last_error(), bytes)


@no_gpu
def test_null_pointers_are_rejected_with_a_message(lib):
    rc = lib.lz_gla_fwd(None, None, None, None, None, 1, 1, 1, 8, 16, 16, 0, 64, None, 0, None)
    refused(lib, rc, b"null")
    rc = lib.lz_swa_fwd(None, None, None, None, 0, None, None, 1, 1, 1, 8, 16, 4, 0.25, None)
    refused(lib, rc, b"null")


@no_gpu
def test_bad_sizes_are_rejected_before_any_launch(lib):
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    # any F, D up to LZ_GLA_MAX_DIM (tiles past the walks' own sizes): F = 5000
    # is refused; F = 300 is not refused for its size (here: for the workspace)
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1, 1, 1, 8, 5000, 16, 0, 64, None, 0, None)
    refused(lib, rc, b"beyond")
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1, 1, 1, 8, 300, 16, 0, 64, None, 0, None)
    refused(lib, rc, b"workspace")
    # entry points that run the walks directly keep their sizes
    rc = lib.lz_gla_prefill(p, p, p, p, p, p, 1, 1, 1, 8, 300, 16, 0, 64, p, 1 << 20, None)
    refused(lib, rc, b"unsupported")
    rc = lib.lz_gla_fwd_noalloc(p, p, p, p, p, 1, 1, 1, 8, 256, 128, 0, 64, None)
    refused(lib, rc, b"unsupported")
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1, 1, 1, 8, 16, 16, 0, 48, None, 0, None)
    refused(lib, rc, b"chunk")
    rc = lib.lz_swa_fwd(p, p, p, p, 65537, p, p, 1, 1, 1, 8, 16, 4, 0.25, None)
    refused(lib, rc, b"n_meta")
    rc = lib.lz_swa_fwd(p, p, p, p, 0, p, p, 1, 1, 1, 8, 512, 4, 0.25, None)
    refused(lib, rc, b"dim")
    rc = lib.lz_swa_fwd(p, p, p, p, 0, p, p, 1, 1, 1, 8, 16, 0, 0.25, None)
    refused(lib, rc, b"window")
    ws = lib.lz_gla_bwd_workspace_bytes(2, 3, 100, 24, 20, 0, 64)
    assert ws > 0
    rc = lib.lz_gla_bwd(p, p, p, p, p, p, p, p, p, 0, 2, 3, 3, 100, 24, 20, 0, 64, None, 0, p,
                        ws - 1, None)
    refused(lib, rc, b"workspace")
    # kv_heads must divide heads (grouped-query operands)
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1, 4, 3, 8, 16, 16, 0, 64, None, 0, None)
    refused(lib, rc, b"kv_heads")
    rc = lib.lz_swa_fwd(p, p, p, p, 0, p, p, 1, 4, 0, 8, 16, 4, 0.25, None)
    refused(lib, rc, b"kv_heads")
    # 32-bit addressing: a (batch, head) slab of fp32 rows under 2 GiB, B*H*L under 2^31
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1, 1, 1, 1 << 21, 256, 64, 0, 64, None, 0, None)
    refused(lib, rc, b"slab")
    rc = lib.lz_gla_fwd(p, p, p, p, p, 1 << 12, 1 << 10, 1 << 10, 1 << 10, 64, 64, 0, 64, None,
                        0, None)
    refused(lib, rc, b"row limit")
    rc = lib.lz_swa_fwd(p, p, p, p, 0, p, p, 1, 1, 1, 1 << 22, 128, 64, 0.25, None)
    refused(lib, rc, b"slab")
    rc = lib.lz_gla_bwd(p, p, p, p, p, p, p, p, p, 0, 1, 1, 1, 1 << 21, 256, 64, 0, 64, None, 0,
                        p, 1, None)
    refused(lib, rc, b"slab")


@no_gpu
def test_gate_mode_bits_are_checked(lib):
    """gate_mode takes LZ_GATE_PER_HEAD (1), LZ_GATE_LOGIT (2) and the hint
    LZ_GLA_NO_REUSE (4) only."""
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    refused(lib, lib.lz_gla_fwd(p, p, p, p, p, 1, 1, 1, 8, 16, 16, 8, 64, None, 0, None),
            b"gate_mode")
    refused(lib, lib.lz_gla_decode_step(p, p, p, p, p, p, 1, 4, 2, 64, 64, 8, None), b"gate_mode")
    ws = lib.lz_gla_bwd_workspace_bytes(1, 1, 8, 16, 16, 3, 64)
    rc = lib.lz_gla_bwd(p, p, p, p, p, p, p, p, p, 0, 1, 1, 1, 8, 16, 16, -1, 64, None, 0, p, ws,
                        None)
    refused(lib, rc, b"gate_mode")
    text = open(HEADER).read()
    assert "#define LZ_GATE_PER_HEAD 1" in text and "#define LZ_GATE_LOGIT 2" in text
    assert "#define LZ_GLA_NO_REUSE 4" in text
    assert (kernels.GATE_PER_HEAD, kernels.GATE_LOGIT, kernels.GLA_NO_REUSE) == (1, 2, 4)


@no_gpu
def test_phi_forward_rejects_bad_arguments(lib):
    """lz_gla_fwd_phi takes head_dim 64 with feature_dim 128 only, and checks
    its pointers, kv heads, gate mode and workspace like lz_gla_fwd."""
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    f = lib.lz_gla_fwd_phi
    # q, wq, fk, v, log_gamma, y, state, B, H, kv_heads, L, head_dim, feature_dim, gate_mode,
    # chunk, workspace, workspace_bytes, stream
    refused(lib, f(p, p, p, p, p, p, None, 1, 4, 2, 64, 32, 128, 0, 64, p, 1 << 20, None),
            b"unsupported")
    refused(lib, f(p, p, p, p, p, p, None, 1, 4, 2, 64, 64, 64, 0, 64, p, 1 << 20, None),
            b"unsupported")
    refused(lib, f(None, p, p, p, p, p, None, 1, 4, 2, 64, 64, 128, 0, 64, p, 1 << 20, None),
            b"null")
    refused(lib, f(p, p, p, p, p, p, None, 1, 4, 3, 64, 64, 128, 0, 64, p, 1 << 20, None),
            b"kv_heads")
    refused(lib, f(p, p, p, p, p, p, None, 1, 4, 2, 64, 64, 128, 8, 64, p, 1 << 20, None),
            b"gate_mode")
    need = lib.lz_gla_fwd_workspace_bytes(1, 4, 4096, 256, 64, 0, 64)
    assert need > 0
    refused(lib, f(p, p, p, p, p, p, None, 1, 4, 2, 4096, 64, 128, 0, 64, p, need - 1, None),
            b"workspace")


@no_gpu
def test_decode_entry_points_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    # lz_swa_decode_step(q, k_cache, v_cache, meta, n_meta, y, B, H, kv_heads, window, dim,
    #                    pos, scale, stream)
    sd = lib.lz_swa_decode_step
    refused(lib, sd(p, p, p, p, 4, None, 1, 4, 2, 64, 64, 0, 0.125, None), b"null")
    refused(lib, sd(p, p, p, p, 4, p, 1, 4, 3, 64, 64, 0, 0.125, None), b"kv_heads")
    refused(lib, sd(p, p, p, p, 4, p, 1, 4, 2, 8193, 64, 0, 0.125, None), b"window")
    refused(lib, sd(p, p, p, p, 4, p, 1, 4, 2, 64, 64, -1, 0.125, None), b"pos")
    refused(lib, sd(p, p, p, p, 4, p, 1, 4, 2, 64, 512, 0, 0.125, None), b"dim")
    refused(lib, sd(p, p, p, p, 65537, p, 1, 4, 2, 64, 64, 0, 0.125, None), b"n_meta")
    # lz_gla_decode_step(fq, fk, v, log_gamma, state, y, B, H, kv_heads, F, D, per_head, stream)
    gd = lib.lz_gla_decode_step
    refused(lib, gd(p, p, p, p, p, p, 1, 4, 3, 64, 64, 0, None), b"kv_heads")
    refused(lib, gd(p, p, p, p, None, p, 1, 4, 2, 64, 64, 0, None), b"null")
    refused(lib, gd(p, p, p, p, p, p, 1, 4, 2, 300, 64, 0, None), b"unsupported")


@no_gpu
def test_layer_entry_points_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    fwd = lib.lz_layer_prologue_fwd
    # B, L, heads, kv_heads, head_dim, feature_dim
    refused(lib, fwd(p, p, p, p, p, p, p, 1, p, p, p, p, p, 1, 2, 40, 4, 3, 32, 8, None), b"multiple of kv_heads")
    refused(lib, fwd(p, p, p, p, p, p, p, 1, p, p, p, p, p, 1, 2, 40, 4, 2, 48, 8, None), b"head_dim")
    refused(lib, fwd(p, p, p, p, p, p, p, 1, p, p, p, p, p, 1, 2, 40, 4, 2, 64, 6, None), b"feature_dim")
    # head_dim 128 x feature_dim 128: bf16 inputs are taken (the fused prologue
    # covers them), fp32 ones refused
    refused(lib, fwd(p, p, p, p, p, p, p, 1, p, p, p, p, p, 0, 2, 40, 4, 2, 128, 128, None),
            b"feature_dim")
    refused(lib, fwd(None, p, p, p, p, p, p, 1, p, p, p, p, p, 1, 2, 40, 4, 2, 32, 8, None), b"null")
    ws = lib.lz_layer_prologue_bwd_workspace_bytes(2, 40, 4, 2, 32, 8)
    assert ws > 0
    rc = lib.lz_layer_prologue_bwd(p, p, p, p, p, p, 1, p, p, p, p, p, None, p, p, p, p, p, 1,
                                   2, 40, 4, 2, 32, 8, p, ws - 1, None)
    refused(lib, rc, b"workspace")
    refused(lib, lib.lz_layer_combine_fwd(p, p, p, p, 1, 2, 4, 40, 12, None), b"multiple of 8")
    cws = lib.lz_layer_combine_bwd_workspace_bytes()
    rc = lib.lz_layer_combine_bwd(p, p, p, p, p, p, 1, 2, 4, 40, 32, p, cws - 1, None)
    refused(lib, rc, b"workspace")


@pytest.mark.parametrize("b, length, heads, kv, hd, f", [
    (2, 40, 4, 2, 32, 8), (4, 4096, 32, 8, 64, 128), (1, 7, 8, 8, 128, 64)])
def test_layer_prologue_workspace_sizes(lib, b, length, heads, kv, hd, f):
    """Partial dW tiles [32 ceil-tiles(f), hd] fp32, a q and a kv one per
    workgroup; the grid is one workgroup per 128-row block of both roles
    together, at most 2 per CU on 256 CUs."""
    blocks = -(-b * length * heads // 128) + -(-b * length * kv // 128)
    grid = min(blocks, 512)
    fp = 32 if f <= 32 else (64 if f <= 64 else 128)
    assert lib.lz_layer_prologue_bwd_workspace_bytes(b, length, heads, kv, hd, f) == \
        4 * 2 * grid * fp * hd


def segments(bh, length, f=64, chunk=64):
    """The library's split of each (b, h) sequence into segments (so that
    B*H*segments fills the GPU: 512 workgroups up to F = 128, 256 beyond,
    where the split is then doubled and each walk takes two segments):
    returns (segments, chunks per segment)."""
    wide = padded(f) > 128
    target = 256 if wide else 512
    nt = -(-length // chunk)
    g = min(max(-(-target // bh), 1), nt)
    if wide and g > 1:
        g = min(2 * g, nt)
    cps = -(-nt // g)
    return -(-nt // cps), cps


def padded(n):
    return next(p for p in (32, 64, 128, 256) if n <= p)


def seg_floats(bh, g, f, d):
    return 0 if g <= 1 else bh * g * (padded(f) * padded(d) + padded(f)) + bh * g


@pytest.mark.parametrize("b, h, length, f, d, per_head", [
    (2, 3, 100, 24, 20, 0), (1, 32, 2048, 64, 64, 0), (16, 32, 2048, 128, 128, 1),
    (4, 16, 1553, 64, 64, 1), (1, 4, 1, 256, 64, 0)])
def test_workspace_sizes(lib, b, h, length, f, d, per_head):
    bh = b * h
    g, _ = segments(bh, length, f)
    assert lib.lz_gla_fwd_workspace_bytes(b, h, length, f, d, per_head, 64) == \
        4 * seg_floats(bh, g, f, d)
    assert lib.lz_gla_bwd_workspace_bytes(b, h, length, f, d, per_head, 64) == \
        4 * (4 * bh * length + 2 * seg_floats(bh, g, f, d) + bh * -(-length // 64))


def test_segment_split():
    assert segments(512, 2048) == (1, 32)       # B*H fills the GPU: one walk per (b, h)
    assert segments(32, 2048) == (16, 2)        # training shape: 16 segments of 2 chunks
    assert segments(64, 1553) == (7, 4)         # ragged: the last segment is shorter
    assert segments(6, 1) == (1, 1)
    assert segments(128, 4096, f=256) == (4, 16)   # config-5 layer shape: 2 segments per walk


def test_swa_workspace_sizes(lib):
    # delta [BH, L] plus dmeta partials [BH * ceil(L/128), n_meta]
    assert lib.lz_swa_bwd_workspace_bytes(1, 32, 2048, 64, 4) == 4 * (32 * 2048 + 32 * 16 * 4)
    assert lib.lz_swa_bwd_workspace_bytes(1, 32, 2048, 64, 0) == 4 * 32 * 2048


def test_python_api_validates_shapes():
    x = torch.zeros(1, 2, 8, 16)
    with pytest.raises(ValueError):
        kernels.gla(x, torch.zeros(1, 2, 8, 12), x, torch.zeros(1, 8))
    with pytest.raises(ValueError):
        kernels.gla(x, x, x, torch.zeros(1, 3, 8))
    with pytest.raises(ValueError):
        kernels.gla(x, x, x, torch.zeros(1, 8), chunk=48)
    with pytest.raises(ValueError):
        kernels.swa(x, x, x, torch.zeros(4), 0)
    with pytest.raises(ValueError):
        kernels.swa(x, x, torch.zeros(1, 2, 8, 8), torch.zeros(4), 4)


def test_python_api_refuses_cpu_tensors():
    x = torch.zeros(1, 2, 8, 16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kernels.gla(x, x, x, torch.zeros(1, 8))
    with pytest.raises(ValueError, match="ROCm GPU"):
        kernels.swa(x, x, x, torch.zeros(4), 4)


def test_missing_library_raises(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load(str(tmp_path / "nope.so"))


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "lizard_reproduction_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), f


def test_internal_wrappers_reject_mismatched_shapes_before_any_launch():
    """The launch wrappers below the operator API (used by the layer) take
    k-side operands with fewer heads; a shape they cannot index is refused
    with ValueError before anything reaches the GPU."""
    from lizard_reproduction_amd import layer
    q = torch.zeros(1, 4, 8, 16)
    k2, v2 = torch.zeros(1, 2, 8, 16), torch.zeros(1, 2, 8, 16)
    with pytest.raises(ValueError, match="Hkv dividing H"):
        kernels.gla_forward(q, torch.zeros(1, 3, 8, 16), v2, torch.zeros(1, 8))
    with pytest.raises(ValueError, match="Hkv dividing H"):
        kernels.swa_forward(q, k2, torch.zeros(1, 2, 9, 16), torch.zeros(4), 4)
    with pytest.raises(ValueError, match="log_gamma"):
        kernels.gla_forward(q, k2, v2, torch.zeros(1, 2, 8))
    with pytest.raises(ValueError, match="dy must be"):
        kernels.gla_backward(q, k2, v2, torch.zeros(1, 8), torch.zeros(1, 2, 8, 16), None,
                             torch.bfloat16)
    # the prologue backward wants per-query-head gradients of the k-side operands
    saved = (None,) * 6 + ((1, 8, 4, 2, 32, 8, 0),)
    per_q = [torch.zeros(1, 4, 8, n) for n in (16, 16, 32, 32, 32)]
    with pytest.raises(ValueError, match="dfk must be"):
        layer.prologue_backward(saved, per_q[0], torch.zeros(1, 2, 8, 16), *per_q[2:])
    with pytest.raises(ValueError, match="dv must be"):
        layer.prologue_backward(saved, *per_q[:4], torch.zeros(1, 2, 8, 32))
    with pytest.raises(ValueError, match="k must be"):
        layer.prologue_forward(torch.zeros(1, 8, 128), torch.zeros(1, 8, 32), torch.zeros(1, 8, 64),
                               torch.zeros(8, 32), torch.zeros(8, 32), None, None, 4, 2)


def test_calls_under_graph_capture_are_refused(monkeypatch):
    """The operator API and the layer refuse to run while the current stream
    is being captured into a HIP graph (their per-call torch allocations and
    the library's first-launch LDS setup have not been cleared for capture),
    before anything touches a GPU."""
    import types

    from lizard_reproduction_amd import layer
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    x = torch.zeros(1, 2, 8, 16)
    with pytest.raises(RuntimeError, match="graph capture"):
        kernels.gla(x, x, x, torch.zeros(1, 8))
    with pytest.raises(RuntimeError, match="graph capture"):
        kernels.swa(x, x, x, torch.zeros(4), 4)
    with pytest.raises(RuntimeError, match="graph capture"):
        kernels.gla_prefill(x, x, x, torch.zeros(1, 8))
    cfg = types.SimpleNamespace(hidden_size=64, num_attention_heads=2, num_key_value_heads=1)
    mod = layer.LizardAttention(cfg, 0, window=8, feature_dim=8)
    cos = torch.ones(8, 32)
    with pytest.raises(RuntimeError, match="graph capture"):
        mod(torch.zeros(1, 8, 64), (cos, cos))
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kernels.gla(x, x, x, torch.zeros(1, 8))


@pytest.mark.parametrize("f, d", [(256, 128), (512, 64), (300, 200), (24, 300), (1024, 128)])
def test_tiled_gla_sizes_have_workspaces(lib, f, d):
    """Sizes past the walks' own run on tiles: the forward and backward
    report workspaces that hold at least the tiles' fp32 partial results."""
    from lizard_reproduction_amd import kernels as k
    assert not k.gla_native(f, d)
    b, h, length = 2, 4, 300
    fw = lib.lz_gla_fwd_workspace_bytes(b, h, length, f, d, 1, 64)
    bw = lib.lz_gla_bwd_workspace_bytes(b, h, length, f, d, 1, 64)
    rows = b * h * length
    assert fw >= rows * 2 * min(d, 128) * 2          # at least a D tile of v and of y
    assert bw >= rows * (2 * f + (d if f > 256 else 0)) * 4   # fp32 sums of dfq, dfk (dv)
    assert lib.lz_gla_fwd_workspace_bytes(b, h, length, 5000, d, 1, 64) == 0


@no_gpu
def test_gla_native_predicate_matches_the_library(lib):
    from lizard_reproduction_amd import kernels as k
    for f in (8, 24, 64, 100, 128, 129, 200, 256, 257):
        for d in (8, 20, 64, 65, 100, 128, 129):
            # the no-allocation forward takes exactly the walks' sizes
            p = ctypes.c_void_p(16)
            rc = lib.lz_gla_fwd_noalloc(p, p, p, p, None, 1, 1, 1, 8, f, d, 0, 64, None)
            msg = lib.lz_last_error()
            refused(lib, rc)
            assert (b"unsupported" not in msg) == k.gla_native(f, d), (f, d, msg)
