#!/usr/bin/env python3
"""Benchmark of the Lizard attention hot path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu-baseline]

Headline (the step that ``value`` and ``ms_per_step`` time): one GLA forward,
``kernels.gla(fq, fk, v, log_gamma)``, at the shape the reference's Table-3
benchmark and the north-star target use (src/benchmark.py:28-41,113-141):
B=16, H=32, L=2048, F=D=128, per-head gate log_gamma = logsigmoid(N(2, 1.5)),
fq, fk = softplus(N(0,1)), v = N(0,1), all bf16 and resident in HBM before
the timed region.  The step is exactly one kernel launch, so the event-timed
average is also the kernel's average duration, the basis of ``roofline``.

Beside it (``extra``), each timed as the median of per-iteration HIP events
after warm-up, like triton.testing.do_bench(return_mode="median") in the
reference (src/benchmark.py:57-66):
  * GLA fwd+bwd at the headline shape (grads reset each iteration; median
    of 100 after 1 s of untimed fwd+bwd and 10 warm-ups, as the forward
    settles below);
  * BASELINE config 2, GLA fwd and fwd+bwd at the training shape (B=1, H=32,
    L=2048, d=64, per-token gate logsigmoid(N(3,1)));
  * BASELINE config 3, SWA fwd and fwd+bwd (B=1, H=32, L=2048, d=64, W=64,
    4 sink logits, RoPE'd q and k);
  * BASELINE config 4 sweep, GLA fwd and fwd+bwd, B in {1,4,16},
    L in {2K,4K,8K,16K}, d=128, per-head gate (skip with --no-sweep); its
    forward rows are timed like the headline (mean of back-to-back launches
    after a short settle), so the B=16 L=2048 row is the headline again;
  * BASELINE config 5, a Llama-3.2-1B-shaped model (hidden 2048, 16 blocks,
    32 query / 8 kv heads, head_dim 64, intermediate 8192, vocab 128256,
    RoPE theta 500000, tied embeddings, random-init bf16 weights) with every
    attention block a LizardAttention (hip backend: feature_dim 128 so F=256,
    D=64, window 64, 4 sinks, per-token gate), one training step's
    forward + cross-entropy backward at B=4, L=4096 on uniform random ids;
    plus one such layer alone (skip with --no-layer).

Clocks: before its warm-up, the headline forward is launched untimed for
--settle-seconds (2 s) of wall time, so that the GPU clocks have settled
whatever --warmup the caller passes; the reported ``warmup`` is the W
untimed steps that follow, as passed.

Also in ``extra``: the algorithmic HBM bytes and HBM fraction of every fwd+bwd
line, and at config 2 the analytic HBM floor of the reference's own
two-kernel design (its per-chunk states and fp32 intermediates through HBM),
the stand-in for its ROCm-Triton build, which cannot run on the GPU box.

``cpu_baseline`` times the dense fp32 PyTorch restatement of the reference's
torch backend (oracle.lizard_oracle: gla_kernel_api, swa_kernel_api and
lizard_layer, the math of src/lizard_attention.py:20-97) on the host cores
(the CPU affinity, capped by a cgroup CPU quota; the count is reported),
median of 5 after one warm-up, after the GPU work: the headline forward (its
``value``) and fwd+bwd on a sample of (b, h) slices at the full L scaled to
all B*H slices (each slice is an independent dense problem), configs 1-3
whole, and one config-5 layer at B=1 (``extra.cpu_baselines``).

``--only NAME`` runs one fwd+bwd workload (headline, config 2, config 3, or
one config-5 layer) --steps times and nothing else, for rocprofv3 runs.

Only one GPU is supported: --gpus N with N > 1 exits with a message.
"""
import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("GLA fwd & fwd+bwd ms + MFMA util% (H=32,d=128,L=2K–16K); "
          "SWA fwd+bwd ms")
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
MFMA_BF16_PEAK_TFS = 2516.6    # MI355X dense bf16 MFMA, vendor figure
CHUNK = 64


def gla_fwd_flops(bh, length, nf, nd):
    """4FD + 2CF + 2CD per token and head: K~^T V, Q~ S, fq fk^T, A V."""
    return bh * length * (4 * nf * nd + 2 * CHUNK * nf + 2 * CHUNK * nd)


def gla_fwd_bwd_flops(bh, length, nf, nd):
    """12FD + 8CF + 6CD per token and head (forward plus the reference's
    backward algorithm, src/kernels/gla.py:104-194)."""
    return bh * length * (12 * nf * nd + 8 * CHUNK * nf + 6 * CHUNK * nd)


def gla_fwd_bytes(bh, length, nf, nd, per_head):
    """Algorithmic HBM bytes of one forward: read fq, fk (F bf16 each), v
    (D bf16), the gate (fp32, per head or shared by the heads of a token),
    write y (D bf16)."""
    gate = 4 if per_head else 0
    return bh * length * (2 * nf + 2 * nf + 2 * nd + 2 * nd + gate)


def swa_weff(length, window):
    return sum(min(i + 1, window) for i in range(length)) / length


def swa_flops(bh, length, d, window, backward):
    return (14 if backward else 4) * d * swa_weff(length, window) * bh * length


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (scaled by a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "gla_fwd_headline_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes"])
    except (OSError, ValueError, KeyError):
        return None


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-sweep", action="store_true", help="skip the config-4 sweep")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=0.5,
                   help="target CPU time of one headline cpu_baseline sample run")
    p.add_argument("--settle-seconds", type=float, default=2.0,
                   help="untimed launches of the headline (or of the --only workload) "
                        "before its warmup, so clocks settle")
    p.add_argument("--only", default=None,
                   choices=["headline_fwd_bwd", "config2", "config3", "config5_layer"],
                   help="run only this workload --steps times (for profiler runs)")
    p.add_argument("--headline-only", action="store_true",
                   help="time only the headline step (for profiler runs)")
    p.add_argument("--no-layer", action="store_true", help="skip the config-5 layer stack")
    p.add_argument("--layer-only", action="store_true",
                   help="run only the config-5 layer stack (for profiling)")
    p.add_argument("--one-layer", action="store_true",
                   help="with --layer-only: only the single-layer part (for profiling)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a plain 1 GiB device copy, the reference kernel that "
                        "scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    return p.parse_args()


def gla_inputs(torch, batch, heads, length, dim, per_head, mean, std, seed=0):
    import torch.nn.functional as F
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (batch, heads, length, dim)
    fq = F.softplus(torch.randn(shape, device="cuda", generator=g)).bfloat16()
    fk = F.softplus(torch.randn(shape, device="cuda", generator=g)).bfloat16()
    v = torch.randn(shape, device="cuda", generator=g).bfloat16()
    gshape = (batch, heads, length) if per_head else (batch, length)
    lg = F.logsigmoid(mean + std * torch.randn(gshape, device="cuda", generator=g))
    dy = torch.randn(shape, device="cuda", generator=g).bfloat16()
    return fq, fk, v, lg, dy


def swa_inputs(torch, batch, heads, length, dim, sinks=4, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (batch, heads, length, dim)
    q, k, v = (torch.randn(shape, device="cuda", generator=g) for _ in range(3))
    inv = 1.0 / (500000.0 ** (torch.arange(0, dim, 2, device="cuda", dtype=torch.float64) / dim))
    ang = torch.outer(torch.arange(length, device="cuda", dtype=torch.float64), inv)
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    half = dim // 2

    def rope(x):
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return (x.double() * cos + rot.double() * sin).bfloat16()
    meta = torch.randn(sinks, device="cuda", generator=g)
    dy = torch.randn(shape, device="cuda", generator=g).bfloat16()
    return rope(q), rope(k), v.bfloat16(), meta, dy


def median_ms(torch, fn, iters, warmup, reset=None):
    """Median of per-iteration event timings (ms) on the current stream."""
    for _ in range(warmup):
        fn()
        if reset:
            reset()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        if reset:
            reset()
        times.append((start, end))
    torch.cuda.synchronize()
    return statistics.median(s.elapsed_time(e) for s, e in times)


def fwd_bwd_fn(torch, op, inputs, dy, extra=()):
    leaves = [t.detach().clone().requires_grad_() for t in inputs]

    def run():
        y = op(*leaves, *extra)
        y.backward(dy)

    def reset():
        for t in leaves:
            t.grad = None
    return run, reset


def layer_stack(torch, steps, warmup, one_layer=False, decode=True):
    """training step (forward, cross-entropy, backward) of
    a Llama-3.2-1B-shaped model whose attention blocks are LizardAttention,
    and of one such layer alone; medians of per-step events.  With
    one_layer, only the single layer (and its decode, unless decode=False)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from lizard_reproduction_amd import _lib, kernels
    from lizard_reproduction_amd.layer import LizardAttention, to_lizard
    cfg = LlamaConfig(hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=64,
                      vocab_size=128256, rope_theta=500000.0, max_position_embeddings=4096,
                      tie_word_embeddings=True, attn_implementation="eager")
    batch, length = 4, 4096
    opts = dict(window=64, num_meta=4, feature_dim=128)
    out = {"shape": "Llama-3.2-1B shape: hidden 2048, 16 blocks, 32 q / 8 kv heads, "
                    "head_dim 64, intermediate 8192, vocab 128256, tied embeddings; "
                    "LizardAttention F=256 D=64 W=64 4 sinks; B=4 L=4096; bf16 random init",
           "intermediate_size_used": 8192}
    torch.manual_seed(0)
    # one layer alone: hidden states in, fwd + bwd with a random upstream grad
    layer = LizardAttention(cfg, 0, **opts).to("cuda", torch.bfloat16)
    with torch.no_grad():
        for p in (layer.W_gamma.weight, layer.meta_tokens):
            p.normal_(0, 0.02)
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    rotary = LlamaRotaryEmbedding(cfg).to("cuda")
    x = torch.randn(batch, length, 2048, device="cuda", dtype=torch.bfloat16)
    pos = torch.arange(length, device="cuda")[None].expand(batch, length)
    rope = rotary(x, pos)
    xg = x.detach().requires_grad_()
    gy = torch.randn_like(x)

    def layer_step():
        y = layer(xg, rope)[0]
        y.backward(gy)

    def layer_reset():
        xg.grad = None
        layer.zero_grad(set_to_none=True)
    with torch.no_grad():
        out["one_layer_fwd_ms"] = round(median_ms(torch, lambda: layer(xg, rope), 5, 2), 3)
    out["one_layer_fwd_bwd_ms"] = round(median_ms(torch, layer_step, max(5, steps), 2,
                                                  layer_reset), 3)
    print(f"[bench] config5 one layer: {out}", file=sys.stderr, flush=True)
    if one_layer and not decode:
        return out

    # layer-level decode: prefill the 4096-token prompts, then one token per
    # sequence through LizardAttention.step (projections, one-token prologue,
    # GLA and SWA decode kernels, blend, o_proj); and the SWA decode kernel
    # alone, 64 back-to-back C-ABI calls between two HIP events
    lib = _lib.load()
    with torch.no_grad():
        out["layer_prefill_ms"] = round(median_ms(torch, lambda: layer.prefill(x, rope), 5, 2), 3)
        _, cache = layer.prefill(x, rope)
        x1 = torch.randn(batch, 1, 2048, device="cuda", dtype=torch.bfloat16)
        rope1 = rotary(x1, torch.full((batch, 1), length, device="cuda"))
        out["layer_decode_step_ms"] = round(
            median_ms(torch, lambda: layer.step(x1, rope1, cache), 20, 5), 4)
        q1 = torch.randn(batch, 32, 64, device="cuda").bfloat16()
        ys1 = torch.empty_like(q1)
        meta = layer.meta_tokens.detach().float().contiguous()
        sargs = [q1.data_ptr(), cache.k.data_ptr(), cache.v.data_ptr(), meta.data_ptr(), 4,
                 ys1.data_ptr(), batch, 32, 8, opts["window"], 64, length, 0.125,
                 torch.cuda.current_stream().cuda_stream]

        def sdec64():
            for _ in range(64):
                lib.lz_swa_decode_step(*sargs)
        out["swa_decode_step_us"] = round(median_ms(torch, sdec64, 5, 2) / 64 * 1e3, 2)
    del layer, xg, gy, rope, rotary, cache, x1, rope1, q1, ys1
    torch.cuda.empty_cache()
    print(f"[bench] config5 layer decode: prefill {out['layer_prefill_ms']} ms, step "
          f"{out['layer_decode_step_ms']} ms, SWA decode kernel {out['swa_decode_step_us']} us",
          file=sys.stderr, flush=True)
    if one_layer:
        return out

    # recurrent decode of the GLA branch at the layer's shape: one token per
    # (b, h) after a 4096-token prefill (state [B, H, F*D + F] fp32 in HBM)
    fq = torch.rand(batch, 32, length, 256, device="cuda").bfloat16()
    fk = torch.rand_like(fq)
    v = torch.randn(batch, 32, length, 64, device="cuda").bfloat16()
    lg = torch.nn.functional.logsigmoid(torch.randn(batch, length, device="cuda") + 3)
    _, state = kernels.gla_prefill(fq, fk, v, lg)
    out["gla_prefill_ms"] = round(median_ms(torch, lambda: kernels.gla_prefill(fq, fk, v, lg),
                                            5, 2), 3)
    # one step = one lz_gla_decode_step launch on contiguous per-token inputs;
    # 64 back-to-back C-ABI calls between two HIP events (the Python wrapper's
    # own checks and casts cost more than the kernel at this size, so they are
    # timed separately)
    tok = [t[:, :, -1].contiguous() for t in (fq, fk, v)]
    lg1 = lg[:, -1].contiguous()
    y1 = torch.empty_like(tok[2])
    args = [t.data_ptr() for t in tok] + [lg1.data_ptr(), state.data_ptr(), y1.data_ptr(),
                                          batch, 32, 32, 256, 64, 0,
                                          torch.cuda.current_stream().cuda_stream]

    def dec64():
        for _ in range(64):
            lib.lz_gla_decode_step(*args)
    t_dec = median_ms(torch, dec64, 5, 2) / 64
    t_py = median_ms(torch, lambda: kernels.gla_decode_step(*tok, lg1, state), 50, 5)
    out["gla_decode_step_us"] = round(t_dec * 1e3, 2)
    out["gla_decode_step_python_us"] = round(t_py * 1e3, 2)
    out["gla_decode_state_gbs"] = round(2 * state.numel() * 4 / (t_dec * 1e-3) / 1e9, 1)
    del fq, fk, v, lg, state, tok, lg1, y1
    torch.cuda.empty_cache()
    print(f"[bench] config5 decode: prefill {out['gla_prefill_ms']} ms, step "
          f"{out['gla_decode_step_us']} us ({out['gla_decode_step_python_us']} us through "
          f"the Python wrapper)", file=sys.stderr, flush=True)

    model = LlamaForCausalLM(cfg).to(torch.bfloat16)
    to_lizard(model, **opts)
    model = model.to("cuda")
    model.train()
    ids = torch.randint(0, cfg.vocab_size, (batch, length), device="cuda")

    def step():
        model(input_ids=ids, labels=ids).loss.backward()

    def reset():
        model.zero_grad(set_to_none=True)
    t = median_ms(torch, step, max(1, steps), max(1, warmup), reset)
    out["model_fwd_bwd_ms"] = round(t, 2)
    out["tokens_per_s"] = round(batch * length / t * 1e3, 1)
    out["peak_hbm_gib"] = round(torch.cuda.max_memory_allocated() / 2**30, 1)
    del model, ids
    torch.cuda.empty_cache()
    print(f"[bench] config5 model: {out}", file=sys.stderr, flush=True)
    return out


def host_cores():
    """Host cores this process may use: its CPU affinity, capped by a cgroup
    CPU quota when one is set (a GPU box's share of a larger host)."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def host_cpu_name():
    name = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return name


def cpu_median_s(fn, reps=5):
    """Median wall time (s) of `reps` calls after one warm-up call."""
    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baselines(torch, cpu_inputs, slice_target_s, with_layer):
    """The reference's torch backend -- its dense L x L PyTorch math
    (src/lizard_attention.py:20-44), restated as oracle.lizard_oracle
    (gla_kernel_api, swa_kernel_api, lizard_layer) -- in fp32 on the host
    cores, median of 5 after one warm-up, fwd and fwd+bwd, on the same
    seeded inputs as the GPU lines.  The headline runs on a sample of its
    B*H (b, h) slices (each slice is an independent dense problem) scaled to
    all of them; configs 1-3 run whole; config 5 runs one layer at B=1,
    median of 3 (the dense layer at B=4 needs ~4x the ~20 GB of B=1; rows are
    independent, so B=4 is 4x the B=1 figure)."""
    from oracle import lizard_oracle as lo
    cores = host_cores()
    torch.set_num_threads(cores)
    out = {"cores": cores, "affinity_cpus": len(os.sched_getaffinity(0)),
           "cpu": host_cpu_name(), "method": "median of 5 after 1 warm-up, fp32"}

    def gla_fb(ins, dy):
        leaves = [t.float().requires_grad_() for t in ins]
        lo.gla_kernel_api(*leaves, dtype=torch.float32).backward(dy.float())

    def swa_fb(ins, dy, window):
        leaves = [t.float().requires_grad_() for t in ins]
        lo.swa_kernel_api(*leaves, window, dtype=torch.float32).backward(dy.float())

    # headline (B=16 H=32 L=2048 F=D=128, per-head gate) on whole (b, h) slices
    fq, fk, v, lg, dy = cpu_inputs["headline"]
    bh = fq.shape[0] * fq.shape[1]
    flat = [t.reshape(bh, 1, *t.shape[2:]) for t in (fq, fk, v, dy)]
    lgf = lg.reshape(bh, 1, lg.shape[-1])

    def sl(n):
        return [t[:n] for t in flat[:3]] + [lgf[:n]], flat[3][:n]
    t0 = time.perf_counter()
    with torch.no_grad():
        lo.gla_kernel_api(*sl(2)[0], dtype=torch.float32)
    per = max((time.perf_counter() - t0) / 2, 1e-4)
    n = int(max(2, min(bh, slice_target_s / per)))
    with torch.no_grad():
        f = cpu_median_s(lambda: lo.gla_kernel_api(*sl(n)[0], dtype=torch.float32))
    fb = cpu_median_s(lambda: gla_fb(*sl(n)))
    out["headline_gla"] = {"fwd_ms": round(f / n * bh * 1e3, 1),
                           "fwd_bwd_ms": round(fb / n * bh * 1e3, 1),
                           "sample": f"{n} of {bh} (b, h) slices at L=2048 F=D=128, scaled "
                                     f"x{bh / n:.1f}"}
    print(f"[bench] cpu headline: {out['headline_gla']}", file=sys.stderr, flush=True)
    # configs 1-3, whole workloads
    for name, key in (("config1_gla_fwd", "config1"), ("config2_gla_train", "config2")):
        fq, fk, v, lg, dy = cpu_inputs[key]
        with torch.no_grad():
            f = cpu_median_s(lambda: lo.gla_kernel_api(fq, fk, v, lg, dtype=torch.float32))
        row = {"fwd_ms": round(f * 1e3, 2)}
        if key == "config2":
            row["fwd_bwd_ms"] = round(cpu_median_s(lambda: gla_fb((fq, fk, v, lg), dy)) * 1e3, 2)
        out[name] = row
    q, k, v, meta, dy = cpu_inputs["config3"]
    with torch.no_grad():
        f = cpu_median_s(lambda: lo.swa_kernel_api(q, k, v, meta, 64, dtype=torch.float32))
    out["config3_swa"] = {"fwd_ms": round(f * 1e3, 2), "fwd_bwd_ms": round(
        cpu_median_s(lambda: swa_fb((q, k, v, meta), dy, 64)) * 1e3, 2)}
    print(f"[bench] cpu configs 1-3: {out['config1_gla_fwd']} {out['config2_gla_train']} "
          f"{out['config3_swa']}", file=sys.stderr, flush=True)
    if with_layer:
        out["config5_one_layer_b1"] = cpu_layer(torch, lo)
        print(f"[bench] cpu config5 layer: {out['config5_one_layer_b1']}", file=sys.stderr,
              flush=True)
    return out


def cpu_layer(torch, lo):
    """One config-5 LizardAttention (hidden 2048, 32 q / 8 kv heads, head_dim
    64, feature_dim 128, W=64, 4 sinks) as the reference's dense torch
    backend computes it (oracle.lizard_layer, src/lizard_attention.py:73-97),
    fp32, B=1, L=4096: fwd and fwd+bwd."""
    import types
    from lizard_reproduction_amd.layer import LizardAttention
    cfg = types.SimpleNamespace(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8)
    torch.manual_seed(0)
    layer = LizardAttention(cfg, 0, window=64, num_meta=4, feature_dim=128)
    params = {n: p.detach().float() for n, p in layer.named_parameters()}
    length = 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, length, 2048, generator=g)
    gy = torch.randn(1, length, 2048, generator=g)
    cos, sin = (t.float()[None] for t in lo.rope_cos_sin(length, 64))

    def fwd():
        with torch.no_grad():
            lo.lizard_layer(params, x, cos, sin, 32, 8, 64)

    def fwd_bwd():
        ps = {n: p.clone().requires_grad_() for n, p in params.items()}
        lo.lizard_layer(ps, x.clone().requires_grad_(), cos, sin, 32, 8, 64).backward(gy)
    return {"fwd_ms": round(cpu_median_s(fwd, 3) * 1e3, 1),
            "fwd_bwd_ms": round(cpu_median_s(fwd_bwd, 3) * 1e3, 1),
            "method": "median of 3 after 1 warm-up (tens of seconds per call)",
            "note": "B=1 L=4096; the B=4 model shape is 4 independent rows (4x), 16 layers"}


def ref_design_bytes(nf, nd, chunk):
    """HBM bytes per (token, head) of the reference's two-kernel GLA design
    (src/kernels/gla.py:213-263), each kernel and torch op reading and
    writing its operands exactly once: the analytic floor of that design.
    Forward: cumsum + expand write G (4); _gla_fwd_h reads fk, v, G and writes
    the per-chunk states S (bf16 F x D) and z (fp32 F) -- F D / C and F / C per
    token; _gla_fwd_o reads fq, fk, v, G, S, z, writes y (bf16), y32 (fp32) and
    den.  Backward: delta = sum dy . y32; _gla_bwd_dh reads fq, dy, den, delta,
    G, writes dS, dz; _gla_bwd_dqkv reads fq, fk, v, dy, G, den, delta, S, z,
    dS, dz and writes fp32 dfq, dfk, dv; dg = sum(fq dfq - fk dfk); the casts
    of the fp32 grads to bf16; the gate gradient's reverse cumsum (4 + 4).
    Returns (forward, backward) bytes."""
    F, D, C = nf, nd, chunk
    st, zz = 2 * F * D / C, 4 * F / C
    gate = 4
    fwd = gate + (2 * F + 2 * D + gate + st + zz) + \
        (2 * F + 2 * F + 2 * D + gate + st + zz + 2 * D + 4 * D + 4)
    bwd = (2 * D + 4 * D + 4) + \
        (2 * F + 2 * D + 4 + 4 + gate + st + zz) + \
        (2 * F + 2 * F + 2 * D + 2 * D + gate + 4 + 4 + 2 * st + 2 * zz + 4 * F + 4 * F + 4 * D) + \
        (2 * F + 4 * F + 2 * F + 4 * F + 4) + \
        (4 * F + 4 * F + 4 * D + 2 * F + 2 * F + 2 * D) + 8
    return fwd, bwd


def gla_fwd_bwd_bytes(bh, length, nf, nd, per_head):
    """Algorithmic HBM bytes of one fwd+bwd: the forward's, then the backward
    reading fq, fk, v, dy and the gate and writing bf16 dfq, dfk, dv and the
    fp32 gate gradient (12F + 10D + 12 per token and head with a per-head
    gate)."""
    gate = 4 if per_head else 0
    return gla_fwd_bytes(bh, length, nf, nd, per_head) + \
        bh * length * (4 * nf + 4 * nd + gate + 4 * nf + 2 * nd + gate)


def swa_fwd_bwd_bytes(bh, length, d):
    """SWA fwd (read q, k, v; write y, lse) + bwd (read q, k, v, dy, lse;
    write dq, dk, dv): 22d + 8 bytes per token and head."""
    return bh * length * (22 * d + 8)


def time_headline(torch, kernels, fq, fk, v, lg, steps, warmup, settle_s=2.0):
    """Event-timed mean of `steps` back-to-back headline forwards on the
    current stream, after launching the same forward untimed for `settle_s`
    seconds of wall time (so the GPU's clocks have settled, whatever the
    driver's --warmup) and then `warmup` more untimed steps."""
    with torch.no_grad():
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(20):
                kernels.gla(fq, fk, v, lg)
            torch.cuda.synchronize()
        for _ in range(warmup):
            kernels.gla(fq, fk, v, lg)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            kernels.gla(fq, fk, v, lg)
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def copy_calibration(torch):
    """A plain 1 GiB device copy (torch's copy_, the runtime's copyBuffer
    kernel): the kernel of known size whose rocprofv3 FETCH_SIZE and
    WRITE_SIZE scale those counters to bytes."""
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    t = median_ms(torch, lambda: dst.copy_(src), 10, 2)
    out = {"bytes_read": src.numel() * 2, "bytes_written": dst.numel() * 2,
           "ms": round(t, 4), "gbs": round(2 * src.numel() * 2 / t / 1e6, 1)}
    print(f"[bench] copy calibration: {out}", file=sys.stderr, flush=True)
    return out


def profile_workload(torch, kernels, name, steps, settle_s):
    """--only NAME: run one workload `steps` times after 3 warm-ups, for
    counter and trace runs (rocprofv3) that should see those kernels alone;
    with settle_s > 0 the workload first runs untimed for that many seconds
    (steady clocks for trace runs; counter runs keep it 0, as every
    dispatch under counters is recorded)."""
    if name == "headline_fwd_bwd":
        ins = gla_inputs(torch, 16, 32, 2048, 128, True, 2.0, 1.5)
        run, reset = fwd_bwd_fn(torch, kernels.gla, ins[:4], ins[4])
    elif name == "config2":
        ins = gla_inputs(torch, 1, 32, 2048, 64, False, 3.0, 1.0)
        run, reset = fwd_bwd_fn(torch, kernels.gla, ins[:4], ins[4])
    elif name == "config3":
        ins = swa_inputs(torch, 1, 32, 2048, 64)
        run, reset = fwd_bwd_fn(torch, kernels.swa, ins[:4], ins[4], (64,))
    elif name == "config5_layer":
        return {"config5_layer": layer_stack(torch, steps, 1, one_layer=True, decode=False)}
    else:
        raise SystemExit(f"unknown --only workload {name!r}")
    settle(torch, run, reset, settle_s)
    t = median_ms(torch, run, steps, 3, reset)
    return {name: {"fwd_bwd_ms": round(t, 4), "steps": steps}}


def settle(torch, run, reset, seconds):
    """Run a fwd+bwd untimed for `seconds` of wall time (steady clocks)."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        run()
        reset()
        torch.cuda.synchronize()


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the Lizard hot path here has no multi-GPU build.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from lizard_reproduction_amd import _lib, kernels
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    torch.manual_seed(0)
    if args.layer_only:
        print(json.dumps({"extra": {"config5_layer_stack": layer_stack(torch, 3, 1,
                                                                       args.one_layer)}}),
              flush=True)
        return
    if args.only:
        extra = profile_workload(torch, kernels, args.only, args.steps, args.settle_seconds)
        if args.copy_calibration:
            extra["copy_calibration"] = copy_calibration(torch)
        print(json.dumps({"extra": extra}), flush=True)
        return

    # ---- headline: GLA forward, B=16 H=32 L=2048 F=D=128, per-head gate -----
    B, H, L, D = 16, 32, 2048, 128
    fq, fk, v, lg, dy = gla_inputs(torch, B, H, L, D, True, 2.0, 1.5)
    cpu_inputs = {"headline": [t.cpu() for t in (fq, fk, v, lg, dy)]}
    ms = time_headline(torch, kernels, fq, fk, v, lg, args.steps, args.warmup,
                       0.0 if args.headline_only else args.settle_seconds)
    flops = gla_fwd_flops(B * H, L, D, D)
    nbytes = gla_fwd_bytes(B * H, L, D, D, True)
    achieved_gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    attainable = min(MFMA_BF16_PEAK_TFS, flops / nbytes * HBM_PEAK_GBS / 1e3)
    print(f"[bench] GLA fwd B={B} H={H} L={L} d={D}: {ms:.4f} ms, {tflops:.1f} TFLOP/s, "
          f"{achieved_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    extra = {"headline_gla_fwd": {
        "ms": round(ms, 4), "tflops": round(tflops, 2), "gbs": round(achieved_gbs, 1),
        "mfma_peak_frac": round(tflops / MFMA_BF16_PEAK_TFS, 4),
        "attainable_tflops": round(attainable, 1),
        "attainable_frac": round(tflops / attainable, 4),
        "flops": flops, "bytes": nbytes,
        "clock_settle_s": 0.0 if args.headline_only else args.settle_seconds}}
    if args.copy_calibration:
        extra["copy_calibration"] = copy_calibration(torch)
    if args.headline_only:
        print(json.dumps({"metric": METRIC, "value": round(ms, 4), "unit": "ms",
                          "ms_per_step": round(ms, 4), "steps": args.steps, "extra": extra}),
              flush=True)
        return

    run, reset = fwd_bwd_fn(torch, kernels.gla, (fq, fk, v, lg), dy)
    settle(torch, run, reset, 0.5 * args.settle_seconds)
    t = median_ms(torch, run, 100, 10, reset)
    f = gla_fwd_bwd_flops(B * H, L, D, D)
    fbb = gla_fwd_bwd_bytes(B * H, L, D, D, True)
    extra["headline_gla_fwd_bwd"] = {
        "ms": round(t, 4), "tflops": round(f / t / 1e9, 2),
        "mfma_peak_frac": round(f / t / 1e9 / MFMA_BF16_PEAK_TFS, 4),
        "algorithmic_bytes": fbb, "gbs": round(fbb / t / 1e6, 1),
        "hbm_frac": round(fbb / t / 1e6 / HBM_PEAK_GBS, 4),
        "hbm_floor_ms": round(fbb / HBM_PEAK_GBS / 1e6, 4)}
    print(f"[bench] GLA fwd+bwd headline: {extra['headline_gla_fwd_bwd']}", file=sys.stderr,
          flush=True)
    del fq, fk, v, lg, dy, run, reset
    torch.cuda.empty_cache()

    # ---- config 1: GLA forward (the reference's CPU-runnable case) -----------
    ins = gla_inputs(torch, 1, 4, 256, 64, False, 3.0, 1.0)
    cpu_inputs["config1"] = [t.cpu() for t in ins]
    with torch.no_grad():
        t_f = median_ms(torch, lambda: kernels.gla(*ins[:4]), 100, 10)
    extra["config1_gla_fwd"] = {"shape": "B=1 H=4 L=256 F=D=64 per-token gate",
                                "fwd_ms": round(t_f, 4)}
    del ins

    # ---- config 2: GLA training shape, per-token gate -----------------------
    fq, fk, v, lg, dy = gla_inputs(torch, 1, 32, 2048, 64, False, 3.0, 1.0)
    cpu_inputs["config2"] = [t.cpu() for t in (fq, fk, v, lg, dy)]
    with torch.no_grad():
        t_f = median_ms(torch, lambda: kernels.gla(fq, fk, v, lg), 100, 10)
    run, reset = fwd_bwd_fn(torch, kernels.gla, (fq, fk, v, lg), dy)
    t_fb = median_ms(torch, run, 100, 10, reset)
    c2b = gla_fwd_bwd_bytes(32, 2048, 64, 64, False)
    rf, rb = ref_design_bytes(64, 64, CHUNK)
    units = 32 * 2048
    extra["config2_gla_train"] = {
        "shape": "B=1 H=32 L=2048 F=D=64 per-token gate", "fwd_ms": round(t_f, 4),
        "fwd_bwd_ms": round(t_fb, 4),
        "fwd_tflops": round(gla_fwd_flops(32, 2048, 64, 64) / t_f / 1e9, 2),
        "fwd_bwd_tflops": round(gla_fwd_bwd_flops(32, 2048, 64, 64) / t_fb / 1e9, 2),
        "algorithmic_bytes": c2b, "hbm_floor_ms": round(c2b / HBM_PEAK_GBS / 1e6, 4),
        "reference_design": {
            "bytes_per_token_head": {"fwd": rf, "bwd": rb},
            "fwd_bwd_bytes": int((rf + rb) * units),
            "hbm_floor_fwd_ms": round(rf * units / HBM_PEAK_GBS / 1e6, 4),
            "hbm_floor_fwd_bwd_ms": round((rf + rb) * units / HBM_PEAK_GBS / 1e6, 4),
            "note": "analytic HBM floor of the reference's two-kernel Triton design "
                    "(src/kernels/gla.py) at this shape; its ROCm-Triton build cannot run "
                    "here (the reference's source may not travel to the GPU box)"}}
    # the same fwd+bwd as back-to-back C-ABI launches without autograd: what
    # the kernels sustain when the host keeps ahead of them (the autograd
    # figure above is bound by torch's host-side cost at this size)
    def gla_launches():
        _, state = kernels.gla_forward(fq, fk, v, lg, keep_state=True)
        kernels.gla_backward(fq, fk, v, lg, dy, state, torch.bfloat16)
    extra["config2_gla_train"]["fwd_bwd_launch_ms"] = round(median_ms(torch, gla_launches, 100, 10), 4)
    print(f"[bench] config2: {extra['config2_gla_train']}", file=sys.stderr, flush=True)
    del fq, fk, v, lg, dy, run, reset

    # ---- config 3: SWA with sinks -------------------------------------------
    q, k, v, meta, dy = swa_inputs(torch, 1, 32, 2048, 64)
    cpu_inputs["config3"] = [t.cpu() for t in (q, k, v, meta, dy)]
    with torch.no_grad():
        t_f = median_ms(torch, lambda: kernels.swa(q, k, v, meta, 64), 100, 10)
    run, reset = fwd_bwd_fn(torch, kernels.swa, (q, k, v, meta), dy, (64,))
    t_fb = median_ms(torch, run, 100, 10, reset)
    swa_bytes = 32 * 2048 * (8 * 64 + 4)
    c3b = swa_fwd_bwd_bytes(32, 2048, 64)
    extra["config3_swa"] = {
        "shape": "B=1 H=32 L=2048 d=64 W=64 4 sinks", "fwd_ms": round(t_f, 4),
        "fwd_bwd_ms": round(t_fb, 4),
        "fwd_tflops": round(swa_flops(32, 2048, 64, 64, False) / t_f / 1e9, 2),
        "fwd_bwd_tflops": round(swa_flops(32, 2048, 64, 64, True) / t_fb / 1e9, 2),
        "fwd_gbs": round(swa_bytes / t_f / 1e6, 1),
        "algorithmic_bytes": c3b, "hbm_floor_ms": round(c3b / HBM_PEAK_GBS / 1e6, 4)}
    def swa_launches():
        _, lse = kernels.swa_forward(q, k, v, meta, 64)
        kernels.swa_backward(q, k, v, meta, lse, dy, 64, torch.bfloat16)
    extra["config3_swa"]["fwd_bwd_launch_ms"] = round(median_ms(torch, swa_launches, 100, 10), 4)
    print(f"[bench] config3: {extra['config3_swa']}", file=sys.stderr, flush=True)
    del q, k, v, meta, dy, run, reset
    torch.cuda.empty_cache()

    # ---- config 4 sweep -----------------------------------------------------
    if not args.no_sweep:
        sweep = []
        for b in (1, 4, 16):
            for length in (2048, 4096, 8192, 16384):
                fq, fk, v, lg, dy = gla_inputs(torch, b, 32, length, 128, True, 2.0, 1.5)
                # forward: mean of back-to-back launches, as the headline
                t_f = time_headline(torch, kernels, fq, fk, v, lg, 20, 3, 0.3)
                run, reset = fwd_bwd_fn(torch, kernels.gla, (fq, fk, v, lg), dy)
                t_fb = median_ms(torch, run, 10, 2, reset)
                ff = gla_fwd_flops(b * 32, length, 128, 128)
                fb = gla_fwd_bwd_flops(b * 32, length, 128, 128)
                row = {"B": b, "L": length, "fwd_ms": round(t_f, 4), "fwd_bwd_ms": round(t_fb, 4),
                       "fwd_tflops": round(ff / t_f / 1e9, 1),
                       "fwd_mfma_frac": round(ff / t_f / 1e9 / MFMA_BF16_PEAK_TFS, 4),
                       "fwd_hbm_frac": round(gla_fwd_bytes(b * 32, length, 128, 128, True) /
                                             t_f / 1e6 / HBM_PEAK_GBS, 4),
                       "fwd_bwd_tflops": round(fb / t_fb / 1e9, 1)}
                sweep.append(row)
                print(f"[bench] sweep {row}", file=sys.stderr, flush=True)
                del fq, fk, v, lg, dy, run, reset
                torch.cuda.empty_cache()
        extra["config4_sweep"] = sweep

    # ---- config 5: layer stack ------------------------------------------------
    if not args.no_layer:
        extra["config5_layer_stack"] = layer_stack(torch, 3, 1)

    # ---- CPU baseline (the GPU is idle from here on) --------------------------
    cpu = None
    if not args.no_cpu_baseline:
        base = cpu_baselines(torch, cpu_inputs, args.cpu_seconds, not args.no_layer)
        extra["cpu_baselines"] = base
        h = base["headline_gla"]
        cpu = {"value": h["fwd_ms"], "unit": "ms", "cores": base["cores"], "kind": "port",
               "sample": (f"dense fp32 torch-backend math (oracle.gla_kernel_api, "
                          f"src/lizard_attention.py:20-31) of the headline forward on "
                          f"{h['sample']}; {base['method']}; {base['cores']} threads "
                          f"({base['affinity_cpus']} CPUs in the affinity mask) on "
                          f"{base['cpu']}; fwd+bwd {h['fwd_bwd_ms']} ms; configs 1-3 and "
                          f"config 5 in extra.cpu_baselines")}

    line = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; distributions of BASELINE configs 2-4)",
        "config": {"workload": "GLA forward, per-head gate, B=16 H=32 L=2048 F=D=128, "
                               "chunk 64 (BASELINE config 4 headline point)",
                   "batch": B, "heads": H, "seq_len": L, "feature_dim": D, "value_dim": D,
                   "gate": "per-head logsigmoid(N(2,1.5))", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(), "kernel": "gla_fwd_kernel<128,128,true,false,false,true>",
                     "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
