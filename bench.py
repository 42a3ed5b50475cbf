"""Selective-scan fwd+bwd benchmark on one MI355X.

Workload (default): selective_scan_fn forward + backward, fp32, batch 8,
dim 1536 (Mamba-130m d_inner), dstate 16, seqlen 2048, variable B/C (one
group), z gate, D skip, delta_bias with softplus; dout ~ N(0,1).  A step is
one forward + backward over that batch with all inputs already in HBM.

Prints one JSON line.  ``value`` is the algorithmic HBM bytes of one
forward + backward (inputs read and outputs written once, no checkpoints or
scratch) divided by the measured time per step, in GB/s.  ``roofline``
describes the dominant kernel, timed with HIP events on the stream it runs
on; ``cpu_baseline`` times the C restatement of the reference's algorithm
(oracle/ss_oracle.c, float64) on the same workload (or its first batch rows)
on this host's cores, and, as ``cpu_baseline.selective_scan_ref``, the
PyTorch oracle on a 96-channel sample of it (its per-step autograd
backward does not scale to the full workload).

``--workload ss_fwd_bwd_b4_d5120_n16_l8192_bf16`` is the bf16 scan (batch 4,
dim 5120, seqlen 8192); ``ss_fwd_bwd_b8_d1536_n32_l2048_f32`` the fp32 one at
dstate 32 (the fast kernels once per 16-state slice).

Other workloads (``--workload``; one JSON line each, reported against the
reference's own op order run on the same GPU, not against the CPU):
  mamba_block_b8_l2048_d1024_bf16   MambaSimple block (d_model 1024, d_inner
      2048, dt_rank 64, dstate 16, conv 4) forward + backward, bf16 weights
      and activations, fp32 A / D, hidden states ~ N(0, 1) of (8, 2048, 1024);
  mamba_block_b1_l32768_d1024_bf16  the same block on one sequence of 32768
      (long-context training: the scan runs in sequence segments);
  causal_lm_24x768_b16_l2048_bf16   CausalLM (24 layers, d_model 768, vocab
      50280) forward in eval mode on token ids of (16, 2048);
  causal_lm_24x768_b1_l32768_bf16   the same model on one sequence of 32768;
  causal_lm_24x768_b8_l2048_train_bf16  a training step of that model (forward,
      cross-entropy, backward, AdamW; dropout 0.15 as configured) on (8, 2048).
``value`` is tokens per second; ``ref_op_order`` gives the same step with
the reference's op sequence (RMSNorm and MambaSimple as PyTorch ops around
SelectiveScanFn, the residual added after each block).
  add_rmsnorm_r32768_d768_bf16   the fused residual add + RMSNorm between
      two blocks of that model (32768 rows of 768, bf16) forward + backward;
      ``value`` is algorithmic GB/s, with a roofline line and a CPU baseline
      as for the scan;
  causal_lm_24x768_b16_decode_bf16   single-token decode of that model for 16
      sequences after a 128-token prompt; ``value`` is tokens per second of
      the step replayed as one HIP graph (the eager step beside it);
      ``..._b1_decode_bf16`` and ``..._b64_decode_bf16``: 1 and 64 sequences.

``--calibrate-copy MIB`` instead times a plain device-to-device copy of MIB
MiB (torch's copy kernel); under ``rocprofv3 --pmc FETCH_SIZE`` /
``WRITE_SIZE`` it gives the factor between those counters and bytes actually
read / written, which scales the scan kernels' counters into ``traffic``.

``--cpu-table`` instead prints one JSON line for each of the three scan
configurations (2 x 64 x 256 fp32, the 8 x 1536 x 2048 fp32 benchmark, 4 x
5120 x 8192 bf16 I/O): the GPU step beside the float64 C oracle and the
PyTorch oracle ``selective_scan_ref`` on this host's cores (a markdown table
of the same on stderr).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload NAME] [--no-cpu]
       python bench.py --calibrate-copy 1024
       python bench.py --cpu-table
"""
import argparse
import json
import os
import sys
import time

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

PEAK_HBM_GBS = 8000.0   # MI355X HBM3E, public spec

WORKLOADS = {
    # name: (batch, dim, dstate, seqlen, dtype, seed)
    "ss_fwd_bwd_b8_d1536_n16_l2048_f32": (8, 1536, 16, 2048, "float32", 1001),
    "ss_fwd_bwd_b4_d5120_n16_l8192_bf16": (4, 5120, 16, 8192, "bfloat16", 1002),
    "ss_fwd_bwd_b8_d1536_n32_l2048_f32": (8, 1536, 32, 2048, "float32", 1006),
}
DEFAULT = "ss_fwd_bwd_b8_d1536_n16_l2048_f32"
MODEL_WORKLOADS = {
    # name: (kind, batch, seqlen, d_model, layers, vocab)
    "mamba_block_b8_l2048_d1024_bf16": ("block", 8, 2048, 1024, 1, 0),
    "mamba_block_b1_l32768_d1024_bf16": ("block", 1, 32768, 1024, 1, 0),
    "causal_lm_24x768_b16_l2048_bf16": ("lm", 16, 2048, 768, 24, 50280),
    "causal_lm_24x768_b1_l32768_bf16": ("lm", 1, 32768, 768, 24, 50280),
    "causal_lm_24x768_b8_l2048_train_bf16": ("lm_train", 8, 2048, 768, 24, 50280),
}

NORM_WORKLOADS = {
    # name: (rows, dim, dtype): the residual add + RMSNorm between two blocks of
    # the 24 x 768 CausalLM at batch 16, seqlen 2048 (32768 token rows)
    "add_rmsnorm_r32768_d768_bf16": (32768, 768, "bfloat16"),
}


def norm_bytes(rows, dim, s):
    """Algorithmic HBM bytes of the fused add + RMSNorm.

    forward: read x, residual; write out, s (4 * rows * dim * s); write rstd
    (rows * 4); read weight.  backward: read s, dout, dresidual_out; write dx
    (4 * rows * dim * s); read rstd; read weight, write dweight.  The
    per-workgroup dweight rows are scratch and are not counted."""
    fwd = 4 * rows * dim * s + rows * 4 + dim * s
    bwd = 4 * rows * dim * s + rows * 4 + 2 * dim * s
    return fwd, bwd


def bench_norm(args):
    """Fused residual add + RMSNorm forward + backward; one JSON line."""
    import torch
    from mamba_amd import _native as nat
    from mamba_amd.ops.rms_norm import prepare_rms_norm_bwd, prepare_rms_norm_fwd

    rows, dim, dtype_name = NORM_WORKLOADS[args.workload]
    dtype = getattr(torch, dtype_name)
    s = 2 if dtype != torch.float32 else 4
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(1005)
    x, r, dout, dres = (torch.randn(rows, dim, generator=gen).to(dtype).to(dev) for _ in range(4))
    w = (0.5 * torch.randn(dim, generator=gen)).to(dtype).to(dev)
    out, sres, dx = (torch.empty(rows, dim, dtype=dtype, device=dev) for _ in range(3))
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    dw = torch.empty(dim, dtype=dtype, device=dev)
    ws = torch.empty(int(nat.load().ss_rmsnorm_bwd_workspace_bytes(rows, dim)), dtype=torch.uint8, device=dev)
    fwd = prepare_rms_norm_fwd(x, w, r, 1e-6, out, sres, rstd)
    bwd = prepare_rms_norm_bwd(sres, w, rstd, dout, dres, dx, dw, ws)
    fname = "rmsnorm_fwd_kernel"
    bname = "rmsnorm_bwd_kernel + rmsnorm_dw_reduce"

    def step():
        fwd()
        bwd()

    def timed(fn, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    warm_up(step, args.warmup)
    ms_per_step = timed(step, args.steps)
    warm_up(fwd, args.warmup)
    f_ms = timed(fwd, args.kernel_reps)
    warm_up(bwd, args.warmup)
    kernel_ms = {fname: f_ms, bname: timed(bwd, args.kernel_reps)}
    print(f"[bench] kernels: " + ", ".join(f"{k} {v * 1e3:.1f} us" for k, v in kernel_ms.items()),
          file=sys.stderr, flush=True)
    fwd_bytes, bwd_bytes = norm_bytes(rows, dim, s)
    gbs = (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e9
    dom = max(kernel_ms, key=kernel_ms.get)
    dom_bytes = fwd_bytes if dom == fname else bwd_bytes
    achieved = dom_bytes / (kernel_ms[dom] * 1e-3) / 1e9
    line = {
        "metric": f"add+RMSNorm fwd+bwd GB/s (% HBM peak), rows {rows}, dim {dim}",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": {torch.float32: "f32", torch.bfloat16: "bf16"}.get(dtype, "f16"),
        "data": "synthetic",
        "config": {"workload": args.workload, "rows": rows, "dim": dim, "residual": True, "prenorm": True,
                   "io_dtype": dtype_name, "weight_dtype": dtype_name},
        "pct_hbm_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "algorithmic_bytes_per_step": fwd_bytes + bwd_bytes,
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kernel_ms.items()},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "bytes_per_launch": dom_bytes},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = norm_cpu_baseline(rows, dim, dtype_name)
        line["cpu_baseline"]["gpu_speedup"] = round(gbs / line["cpu_baseline"]["value"], 1)
    print(json.dumps(line), flush=True)


def norm_cpu_baseline(rows, dim, dtype_name, sample_rows=None, reps=3):
    """The oracle's add + RMSNorm (PyTorch on this host's cores, fp32 compute from
    the I/O dtype) forward + autograd backward on `sample_rows` rows (all of
    them by default: well under a second), scaled with the same byte formula."""
    import torch
    from oracle.mamba_block_ref import add_rms_norm_ref

    sample_rows = rows if sample_rows is None else sample_rows

    threads = cpu_threads()
    torch.set_num_threads(threads)
    dtype = getattr(torch, dtype_name)
    gen = torch.Generator().manual_seed(1005)
    x, r, dout, dres = (torch.randn(sample_rows, dim, generator=gen).to(dtype) for _ in range(4))
    w = (0.5 * torch.randn(dim, generator=gen)).to(dtype)

    def run():
        xg, rg, wg = (t.clone().requires_grad_(True) for t in (x, r, w))
        out, s = add_rms_norm_ref(xg, rg, wg)
        torch.autograd.backward([out, s], [dout, dres])

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    s = 2 if dtype != torch.float32 else 4
    fb, bb = norm_bytes(sample_rows, dim, s)
    return {"value": round((fb + bb) / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{sample_rows} of {rows} rows, dim {dim}, {dtype_name}; median of {reps}",
            "seconds_per_sample": round(t, 4)}

DECODE_WORKLOADS = {
    # name: (batch, prompt, d_model, layers, vocab)
    "causal_lm_24x768_b16_decode_bf16": (16, 128, 768, 24, 50280),
    "causal_lm_24x768_b1_decode_bf16": (1, 128, 768, 24, 50280),
    "causal_lm_24x768_b64_decode_bf16": (64, 128, 768, 24, 50280),
}


def bench_decode(args):
    """CausalLM single-token decode (after a prompt prefill); one JSON line.
    ``value`` is tokens per second of the graph-replayed step; the eager
    step (one launch per kernel from Python) is reported beside it."""
    import torch
    from mamba_amd.models import CausalLM, CausalLMConfig, GraphedStep

    batch, prompt, d_model, layers, vocab = DECODE_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.manual_seed(1006)
    cfg = CausalLMConfig(vocab_size=vocab, model_dim=d_model, state_dim=16, conv_kernel=4,
                         expansion_factor=2, num_layers=layers)
    model = CausalLM(cfg, device=dev, dtype=torch.bfloat16).eval()
    ids = torch.randint(0, vocab, (batch, prompt), device=dev)
    cache = model.allocate_inference_cache(batch)
    with torch.no_grad():
        model(ids, inference_cache=cache)
    tok = ids[:, -1].clone()

    def timed(fn, n):
        warm_up(fn, args.warmup)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    with torch.no_grad():
        ms_eager = timed(lambda: model.step(tok, cache), args.steps)
    graphed = GraphedStep(model, cache, batch)
    ms_graph = timed(lambda: graphed(tok), args.steps)
    line = {"metric": f"CausalLM decode tokens/s, {layers} layers, d_model {d_model}, batch {batch}",
            "value": round(batch / (ms_graph * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_graph, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic, random init",
            "config": {"workload": args.workload, "batch": batch, "prompt": prompt, "d_model": d_model,
                       "layers": layers, "vocab": vocab, "dtype": "bf16 (A, D fp32, state fp32)"},
            "eager_step": {"ms_per_step": round(ms_eager, 4), "value": round(batch / (ms_eager * 1e-3), 1),
                           "what": "the same step launched kernel by kernel from Python"},
            "reference": "no decode path (CausalLM.generate is a stub)"}
    print(json.dumps(line), flush=True)


def bench_model(args):
    """Mamba block fwd+bwd or CausalLM forward; one JSON line."""
    import torch
    from mamba_amd.models import CausalLM, CausalLMConfig
    from mamba_amd.modules import MambaSimple

    kind, batch, seqlen, d_model, layers, vocab = MODEL_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    dt = torch.bfloat16
    torch.manual_seed(1003)

    def timed(fn):
        warm_up(fn, args.warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    if kind == "block":
        block = MambaSimple(d_model, state_dim=16, conv_kernel=4, expansion_factor=2, device=dev, dtype=dt)
        x = torch.randn(batch, seqlen, d_model, device=dev, dtype=dt).requires_grad_(True)
        dout = torch.randn(batch, seqlen, d_model, device=dev, dtype=dt)
        params = [x] + list(block.parameters())

        def step():
            return torch.autograd.grad(block(x), params, dout)

        ms = timed(step)
        block.use_fast_path = False
        ms_ref = timed(step) if not args.no_ref_order else None
        metric = f"Mamba block fwd+bwd tokens/s, d_model {d_model}, seqlen {seqlen}"
        config = {"workload": args.workload, "batch": batch, "seqlen": seqlen, "d_model": d_model,
                  "d_inner": 2 * d_model, "dt_rank": block.delta_rank, "dstate": 16, "d_conv": 4,
                  "dtype": "bf16 (A, D fp32)"}
    elif kind == "lm_train":
        cfg = CausalLMConfig(vocab_size=vocab, model_dim=d_model, state_dim=16, conv_kernel=4,
                             expansion_factor=2, num_layers=layers)
        model = CausalLM(cfg, device=dev, dtype=dt).train()
        ids = torch.randint(0, vocab, (batch, seqlen + 1), device=dev)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-4)

        def step():
            logits = model(ids[:, :-1])
            loss = torch.nn.functional.cross_entropy(logits.reshape(-1, vocab).float(), ids[:, 1:].reshape(-1))
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            return loss

        ms = timed(step)
        for layer in model.layers:
            layer.mamba.use_fast_path = False
            layer.norm.use_fast_path = False
        model.norm.use_fast_path = False
        ms_ref = timed(step) if not args.no_ref_order else None
        metric = f"CausalLM training tokens/s, {layers} layers, d_model {d_model}, seqlen {seqlen}"
        config = {"workload": args.workload, "batch": batch, "seqlen": seqlen, "d_model": d_model,
                  "layers": layers, "vocab": vocab, "dtype": "bf16 (A, D fp32)",
                  "step": "forward, cross-entropy, backward, AdamW", "dropout": cfg.dropout_rate}
    else:
        cfg = CausalLMConfig(vocab_size=vocab, model_dim=d_model, state_dim=16, conv_kernel=4,
                             expansion_factor=2, num_layers=layers)
        model = CausalLM(cfg, device=dev, dtype=dt).eval()
        ids = torch.randint(0, vocab, (batch, seqlen), device=dev)

        def step():
            with torch.no_grad():
                return model(ids)

        ms = timed(step)
        for layer in model.layers:
            layer.mamba.use_fast_path = False
            layer.norm.use_fast_path = False
        model.norm.use_fast_path = False
        ms_ref = timed(step) if not args.no_ref_order else None
        metric = f"CausalLM forward tokens/s, {layers} layers, d_model {d_model}, seqlen {seqlen}"
        config = {"workload": args.workload, "batch": batch, "seqlen": seqlen, "d_model": d_model,
                  "layers": layers, "vocab": vocab, "dtype": "bf16 (A, D fp32)", "mode": "eval"}
    tokens = batch * seqlen
    line = {"metric": metric, "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic, random init",
            "config": config,
            "ref_op_order": None if ms_ref is None else {
                "ms_per_step": round(ms_ref, 4), "value": round(tokens / (ms_ref * 1e-3), 1),
                "speedup": round(ms_ref / ms, 3),
                "what": "the reference's op sequence (RMSNorm and MambaSimple as PyTorch ops around "
                        "SelectiveScanFn on the same HIP scan, residual added after each block), "
                        "same weights and inputs"}}
    print(json.dumps(line), flush=True)


def synthetic_inputs(batch, dim, dstate, seqlen, *, seed, dtype):
    """Seeded synthetic scan inputs of the benchmark distributions.

    A CPU generator seeded with ``seed`` draws, in this order, u, delta, z,
    B, C (variable, one group), dt and dout, each N(0, 1) fp32 (dt uniform
    on [1e-3, 1e-1]); delta_bias = dt + log(-expm1(-dt)) is the inverse
    softplus of dt (the form of modules/mamba_simple.py:76); A = -(1..N) per
    channel (modules/mamba_simple.py:80-82,128); D = ones.  The sequence
    tensors are cast to ``dtype``; A, D and delta_bias stay fp32."""
    import torch
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, seqlen, generator=g)
    delta = torch.randn(batch, dim, seqlen, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g)
    B = torch.randn(batch, 1, dstate, seqlen, generator=g)
    C = torch.randn(batch, 1, dstate, seqlen, generator=g)
    dt = torch.rand(dim, generator=g) * (1e-1 - 1e-3) + 1e-3
    dout = torch.randn(batch, dim, seqlen, generator=g)
    return dict(u=u.to(dtype), delta=delta.to(dtype), z=z.to(dtype), B=B.to(dtype), C=C.to(dtype),
                dout=dout.to(dtype), delta_bias=dt + torch.log(-torch.expm1(-dt)),
                A=-torch.arange(1, dstate + 1, dtype=torch.float32).repeat(dim, 1), D=torch.ones(dim))


def kernel_sources_digest():
    """sha256 of the sources the scan kernels are built from: a stored
    traffic figure is only reported while it matches."""
    import hashlib
    h = hashlib.sha256()
    for name in ("ss_fwd.hip", "ss_bwd.hip", "ss_device.hpp", "ss_kernels.hpp", "ss_api.hip"):
        with open(os.path.join(_HERE, "mamba_amd", "csrc", name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()


def stored_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from profiles/traffic_<workload>.json
    (rocprofv3 FETCH_SIZE / WRITE_SIZE, scaled by a copy calibration), with
    where it came from; (None, reason) when there is none or it was taken
    with other kernel sources than the ones built now."""
    path = os.path.join("profiles", f"traffic_{workload}.json")
    full = os.path.join(_HERE, path)
    if not os.path.exists(full):
        return None, f"no {path}"
    with open(full) as f:
        rec = json.load(f)
    if rec.get("sources_sha256") != kernel_sources_digest():
        return None, f"{path} was measured with other kernel sources (stale)"
    if kernel not in rec:
        return None, f"{path} has no entry for {kernel}"
    return rec[kernel], (f"{path}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel build "
                         f"(sources sha256 {rec['sources_sha256'][:12]}), scaled by a 1 GiB copy calibration")


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_threads():
    """Host threads for the CPU baselines: every core this process may run
    on, capped by OMP_NUM_THREADS when that is set (a multi-GPU host that
    gives each GPU's process a share of its cores sets it to that share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def warm_up(fn, steps, min_ms=100.0):
    """Runs fn at least `steps` times and for at least `min_ms` of GPU time:
    the clocks ramp up under sustained load (about 50 ms from idle)."""
    import torch
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        fn()
        torch.cuda.synchronize()


def algorithmic_bytes(batch, dim, dstate, seqlen, s, groups=1):
    """HBM bytes that one forward / backward must move at minimum.

    forward: read u, delta, z; write out (4 * BDL * s); read B, C
    (2 * BGNL * s); read A, D, delta_bias.
    backward: read u, delta, z, dout; write du, ddelta, dz (7 * BDL * s);
    read B, C (2 * BGNL * s) and write fp32 dB, dC (2 * BGNL * 4); read A,
    D, delta_bias and write dA, dD, ddelta_bias.
    """
    BDL = batch * dim * seqlen
    BGNL = batch * groups * dstate * seqlen
    fwd = 4 * BDL * s + 2 * BGNL * s + dim * dstate * 4 + 2 * dim * 4
    bwd = 7 * BDL * s + 2 * BGNL * s + 2 * BGNL * 4 + 2 * dim * dstate * 4 + 4 * dim * 4
    return fwd, bwd


def cpu_baseline(dtype_name, batch, dim, seqlen, dstate, max_seconds=30.0, seed=1001):
    """Times the C restatement of the reference's algorithm (oracle/ss_oracle.c:
    the reference kernels' arithmetic in float64, plain loops) forward +
    backward on this host's cores: one task per (batch row, 96-channel slice),
    run by a pool of cpu_threads() threads (the C calls release the GIL).  A
    one-slice calibration run estimates the time; the sample is the whole
    workload when that takes at most `max_seconds`, else its first batch
    rows.  GB/s uses the same byte formula (and I/O dtype) as ``value``."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    from oracle import c_oracle

    threads = cpu_threads()
    # tasks of at most 96 channels (a divisor of dim when there is one)
    slice_ch = next((k for k in (96, 80, 64, 48, 32, 16) if dim % k == 0), dim)
    x = {k: (v.double() if v is not None else None)
         for k, v in synthetic_inputs(batch, dim, dstate, seqlen, seed=seed, dtype=torch.float32).items()}

    def task(bi, lo):
        hi = lo + slice_ch
        ch = lambda t: t[bi:bi + 1, lo:hi].contiguous()
        u, dl, z, do = ch(x["u"]), ch(x["delta"]), ch(x["z"]), ch(x["dout"])
        A, D, bias = x["A"][lo:hi].contiguous(), x["D"][lo:hi].contiguous(), x["delta_bias"][lo:hi].contiguous()
        B, C = x["B"][bi:bi + 1].contiguous(), x["C"][bi:bi + 1].contiguous()
        c_oracle.fwd(u, dl, A, B, C, D, z=z, delta_bias=bias, delta_softplus=True)
        c_oracle.bwd(u, dl, A, B, C, D, z=z, delta_bias=bias, delta_softplus=True, dout=do)

    t0 = time.perf_counter()
    task(0, 0)
    per_task = time.perf_counter() - t0
    tasks_per_row = dim // slice_ch
    rows = batch
    while rows > 1 and rows * tasks_per_row * per_task / threads > max_seconds:
        rows //= 2
    tasks = [(bi, k * slice_ch) for bi in range(rows) for k in range(tasks_per_row)]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(lambda a: task(*a), tasks))
    dt = time.perf_counter() - t0
    print(f"[bench] cpu C oracle: {len(tasks)} tasks of {slice_ch} channels on {threads} threads: {dt:.2f} s",
          file=sys.stderr, flush=True)
    s = 2 if dtype_name != "float32" else 4
    fwd_b, bwd_b = algorithmic_bytes(rows, dim, dstate, seqlen, s)
    return {
        "value": round((fwd_b + bwd_b) / dt / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"oracle/ss_oracle.c (float64 C restatement of the reference kernels) fwd+bwd on batch {rows} "
                  f"x dim {dim} x seqlen {seqlen} x dstate {dstate}, {len(tasks)} tasks of {slice_ch} channels "
                  f"on {threads} threads, {dt:.2f} s; same byte formula as value",
        "elems_per_s": round(rows * dim * seqlen / dt, 1),
        "seconds": round(dt, 3),
    }


def cpu_ref_sample(dtype_name, seqlen, dstate, batch=1, dim=96, reps=3, seed=1001):
    """Times the PyTorch oracle ``selective_scan_ref`` (a per-step loop in
    fp32 with autograd for the backward) on this host's cores, forward
    (no_grad) and forward + backward, on a bounded sample: `batch` rows of
    `dim` channels at the workload's dstate and the given seqlen (its backward
    through the per-step graph grows faster than the sample: 96 channels of
    2048 steps take seconds, 1536 channels far more than a bench run may
    spend, and so do longer sequences).  Median of
    `reps` after one warm-up; GB/s by the same byte formula as ``value``."""
    import torch
    from oracle.selective_scan_ref import selective_scan_ref

    threads = cpu_threads()
    torch.set_num_threads(threads)
    x = synthetic_inputs(batch, dim, dstate, seqlen, seed=seed, dtype=torch.float32)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    g = {k: x[k].clone().requires_grad_(True) for k in names}
    args = lambda: (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"])

    def fwd():
        with torch.no_grad():
            selective_scan_ref(*args(), z=g["z"], delta_bias=g["delta_bias"], delta_softplus=True)

    def fwd_bwd():
        out = selective_scan_ref(*args(), z=g["z"], delta_bias=g["delta_bias"], delta_softplus=True)
        torch.autograd.grad(out, [g[k] for k in names], x["dout"])

    times = {}
    for name, fn in (("fwd", fwd), ("fwd_bwd", fwd_bwd)):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        times[name] = sorted(ts)[len(ts) // 2]
    s = 2 if dtype_name != "float32" else 4
    fwd_b, bwd_b = algorithmic_bytes(batch, dim, dstate, seqlen, s)
    print(f"[bench] cpu selective_scan_ref: batch {batch} x dim {dim}: fwd {times['fwd']:.3f} s, "
          f"fwd+bwd {times['fwd_bwd']:.3f} s on {threads} threads", file=sys.stderr, flush=True)
    return {
        "value": round((fwd_b + bwd_b) / times["fwd_bwd"] / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "fwd_s": round(times["fwd"], 4),
        "fwd_bwd_s": round(times["fwd_bwd"], 4),
        "sample": f"oracle/selective_scan_ref.py (the PyTorch oracle, fp32, autograd backward) on batch {batch} "
                  f"x dim {dim} x seqlen {seqlen} x dstate {dstate}: median of {reps} after one warm-up; "
                  f"same byte formula as value",
    }


def time_copy(mib, reps=5):
    """Copies `mib` MiB device to device `reps` times; (bytes copied, ms per copy)."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return n * 4, ms


# The three scan configurations with the CPU baselines beside the GPU step:
# (label, batch, dim, dstate, seqlen, dtype, seed, (batch, dim, seqlen) of
# the selective_scan_ref sample or None for the whole configuration; its
# per-step autograd graph makes 8192 steps take minutes, so the bf16 case is
# sampled over its first 2048 steps)
CPU_TABLE = [
    ("2 x 64 x 256, fp32 (the CPU-runnable case)", 2, 64, 16, 256, "float32", 1000, None),
    ("8 x 1536 x 2048, fp32 (the benchmark)", 8, 1536, 16, 2048, "float32", 1001, (1, 96, 2048)),
    ("4 x 5120 x 8192, bf16 I/O", 4, 5120, 16, 8192, "bfloat16", 1002, (1, 96, 2048)),
]


def gpu_step_ms(batch, dim, dstate, seqlen, dtype_name, seed, steps, warmup):
    """ms per selective_scan_fn forward + autograd backward on cuda:0 (the
    step ``value`` times), inputs resident in HBM."""
    import torch
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn

    dev = torch.device("cuda:0")
    x = synthetic_inputs(batch, dim, dstate, seqlen, seed=seed, dtype=getattr(torch, dtype_name))
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    g = {k: x[k].to(dev).requires_grad_(True) for k in names}
    dout = x["dout"].to(dev)

    def step():
        out = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                delta_bias=g["delta_bias"], delta_softplus=True)
        return torch.autograd.grad(out, [g[k] for k in names], dout)

    warm_up(step, warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_cpu_table(args):
    """One JSON line per scan configuration: the GPU step beside the float64 C
    oracle (the whole configuration, or its first batch rows past 30 s) and
    the PyTorch oracle selective_scan_ref (whole, or a sample of 96 channels
    of one batch row), all GB/s by the same byte formula; a markdown table of
    the same on stderr."""
    rows = []
    for label, batch, dim, dstate, seqlen, dtype_name, seed, sample in CPU_TABLE:
        s = 2 if dtype_name != "float32" else 4
        fwd_b, bwd_b = algorithmic_bytes(batch, dim, dstate, seqlen, s)
        print(f"[bench] cpu table: {label}", file=sys.stderr, flush=True)
        ms = gpu_step_ms(batch, dim, dstate, seqlen, dtype_name, seed, args.steps, args.warmup)
        c = cpu_baseline(dtype_name, batch, dim, seqlen, dstate, seed=seed)
        rb, rd, rl = sample if sample else (batch, dim, seqlen)
        r = cpu_ref_sample(dtype_name, rl, dstate, batch=rb, dim=rd, seed=seed)
        line = {"config": label, "batch": batch, "dim": dim, "dstate": dstate, "seqlen": seqlen,
                "io_dtype": dtype_name, "gpu_ms_per_step": round(ms, 4),
                "gpu_gbs": round((fwd_b + bwd_b) / (ms * 1e-3) / 1e9, 2),
                "gpu_pct_hbm_peak": round(100.0 * (fwd_b + bwd_b) / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
                "c_oracle": c, "selective_scan_ref": dict(r, sample_shape=f"batch {rb} x dim {rd} x seqlen {rl}")}
        print(json.dumps(line), flush=True)
        rows.append(line)
    print("| configuration | GPU step (ms) | GPU GB/s (% of 8 TB/s) | C oracle (s, GB/s, threads) "
          "| selective_scan_ref fwd / fwd+bwd (s, sample, GB/s) |", file=sys.stderr)
    print("|---|---|---|---|---|", file=sys.stderr)
    for ln in rows:
        c, r = ln["c_oracle"], ln["selective_scan_ref"]
        print(f"| {ln['config']} | {ln['gpu_ms_per_step']:.4f} | {ln['gpu_gbs']:.1f} ({ln['gpu_pct_hbm_peak']:.2f} %) "
              f"| {c['seconds']:.3f} s, {c['value']:.3f} GB/s, {c['cores']} | {r['fwd_s']:.3f} / "
              f"{r['fwd_bwd_s']:.3f} s, {r['sample_shape']}, {r['value']:.4f} GB/s |", file=sys.stderr, flush=True)


def calibrate_copy(mib, reps=5):
    """Copies `mib` MiB device to device `reps` times; prints one JSON line."""
    nbytes, ms = time_copy(mib, reps)
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "ms": round(ms, 5),
                      "GB/s (read + write)": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # scan workloads: 100 + 100 steps by default.  The GPU's clocks ramp under
    # sustained load: after idle the first ~60 steps of the fp32 workload run
    # up to 20 % slower than the settled rate, so a short warm-up would time
    # the ramp rather than the kernels (about 50 ms for each phase here).
    ap.add_argument("--steps", type=int, default=None, help="timed steps (scan 100, other workloads 20)")
    ap.add_argument("--warmup", type=int, default=None, help="warm-up steps (scan 100, other workloads 5)")
    ap.add_argument("--workload", default=DEFAULT,
                    choices=sorted(WORKLOADS) + sorted(MODEL_WORKLOADS) + sorted(NORM_WORKLOADS)
                    + sorted(DECODE_WORKLOADS))
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-ref-order", action="store_true",
                    help="block / LM workloads: skip timing the reference's op order")
    ap.add_argument("--cpu-table", action="store_true",
                    help="only the three scan configurations with the CPU baselines beside the GPU step")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only time a plain device copy of MIB MiB (counter calibration)")
    args = ap.parse_args()
    scan = args.workload in WORKLOADS
    if args.steps is None:
        args.steps = 100 if scan else 20
    if args.warmup is None:
        args.warmup = 100 if scan else 5
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: the benchmark runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the selective scan would shard by batch or channel "
              "with one exchange of dA / dD / delta-bias (or dB / dC) gradients, which is not built here.",
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.cpu_table:
        bench_cpu_table(args)
        return
    if args.workload in MODEL_WORKLOADS:
        bench_model(args)
        return
    if args.workload in NORM_WORKLOADS:
        bench_norm(args)
        return
    if args.workload in DECODE_WORKLOADS:
        bench_decode(args)
        return

    import torch
    from mamba_amd import selective_scan as ss
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn

    batch, dim, dstate, seqlen, dtype_name, seed = WORKLOADS[args.workload]
    dtype = getattr(torch, dtype_name)
    s = 2 if dtype != torch.float32 else 4
    dev = torch.device("cuda:0")
    x = synthetic_inputs(batch, dim, dstate, seqlen, seed=seed, dtype=dtype)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    g = {k: x[k].to(dev).requires_grad_(True) for k in names}
    dout = x["dout"].to(dev)
    params = [g[k] for k in names]

    def step():
        out = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                delta_bias=g["delta_bias"], delta_softplus=True)
        return torch.autograd.grad(out, params, dout)

    warm_up(step, args.warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps
    print(f"[bench] {args.steps} steps: {ms_per_step:.4f} ms/step (wall {wall:.3f} s)", file=sys.stderr, flush=True)

    # ---- per-kernel durations: HIP events on the current stream, which is
    # the stream the library launches on
    with torch.no_grad():
        u, dl, A, B, C, D, z, bias = (g[k].detach() for k in names)
        out = torch.empty_like(dl)
        xck = torch.empty((batch, ss.n_chunks(seqlen), dim, dstate), dtype=torch.float32, device=dev)
        y = torch.empty_like(dl)
        du, dd, dz = torch.empty_like(u), torch.empty_like(dl), torch.empty_like(z)
        dA = torch.zeros(A.shape, dtype=torch.float32, device=dev)
        dB = torch.zeros(B.shape, dtype=torch.float32, device=dev)
        dC = torch.zeros(C.shape, dtype=torch.float32, device=dev)
        dD = torch.zeros(D.shape, dtype=torch.float32, device=dev)
        db = torch.zeros(bias.shape, dtype=torch.float32, device=dev)

        # prepared launches: the arguments are checked once, so back-to-back
        # launches keep the GPU busy and the events time the kernels alone
        fwd = ss.prepare_forward(u, dl, A, B, C, D, bias, True, out, xck, z=z, y=y)
        bwd = ss.prepare_backward(u, dl, A, B, C, D, bias, dout, xck, True, du, dd, dA, dB, dC, dD, db,
                                  z=z, y=y, dz=dz, zero_grads=True)

        tname = {torch.float32: "float", torch.bfloat16: "bf16", torch.float16: "half"}[dtype]
        fname = ss.forward_kernel_name(u, dl, A, B, C, D, bias, True, out, xck, z=z, y=y)
        bname = ss.backward_kernel_name(u, dl, A, B, C, D, bias, dout, xck, True, du, dd, dA, dB, dC, dD, db,
                                        z=z, y=y, dz=dz)
        ws = ss.workspace_bytes(u, dl, A, B, C, D, bias, dout, xck, True, du, dd, dA, dB, dC, dD, db,
                                z=z, y=y, dz=dz)
        fname, bname = f"{fname}<{tname}, z>", f"{bname}<{tname}, z>"
        # dstate 16 S: the fast kernels once per 16-state slice, with two fp32
        # accumulators of batch x dim x seqlen floats in the workspace
        passes = dstate // 16 if dstate > 16 and dstate % 16 == 0 else 1
        acc = 2 * batch * dim * seqlen * 4 if passes > 1 else 0
        if passes > 1:
            fname, bname = f"{fname} x {passes} state slices", f"{bname} x {passes} state slices"
        # zero_grads: a fill launch clears the accumulators (and any dB / dC
        # slices) before the scan; with slices, a last launch sums them
        bname = f"ss_zero_segs + {bname}" + (" + ss_ws_reduce" if ws - acc > 0 else "")
        kernel_ms = {}
        # the set-up above leaves the GPU idle and its clocks drop: warm the
        # prepared launches up as long as the steps, then time each kernel
        warm_up(lambda: (fwd(), bwd()), args.warmup)
        for name, fn in ((fname, fwd), (bname, bwd)):
            fn()
            torch.cuda.synchronize()
            a, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(args.kernel_reps):
                fn()
            b_.record()
            torch.cuda.synchronize()
            kernel_ms[name] = a.elapsed_time(b_) / args.kernel_reps
    print(f"[bench] kernels: " + ", ".join(f"{k} {v * 1e3:.1f} us" for k, v in kernel_ms.items()),
          file=sys.stderr, flush=True)

    fwd_bytes, bwd_bytes = algorithmic_bytes(batch, dim, dstate, seqlen, s)
    total = fwd_bytes + bwd_bytes
    gbs = total / (ms_per_step * 1e-3) / 1e9
    dom = max(kernel_ms, key=kernel_ms.get)
    dom_bytes = fwd_bytes if dom == fname else bwd_bytes
    achieved = dom_bytes / (kernel_ms[dom] * 1e-3) / 1e9

    traffic, traffic_source = stored_traffic(args.workload, dom)

    line = {
        "metric": f"selective-scan fwd+bwd GB/s (% HBM peak) + elems/s, D={dim} N={dstate} L={seqlen}",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dtype == torch.float32 else ("bf16" if dtype == torch.bfloat16 else "f16"),
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": batch, "dim": dim, "dstate": dstate,
                   "seqlen": seqlen, "n_groups": 1, "z_gate": True, "D_skip": True,
                   "delta_softplus": True, "io_dtype": dtype_name},
        "pct_hbm_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "elems_per_s": round(batch * dim * seqlen / (ms_per_step * 1e-3), 1),
        "elem_states_per_s": round(batch * dim * seqlen * dstate / (ms_per_step * 1e-3), 1),
        "algorithmic_bytes_per_step": total,
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kernel_ms.items()},
        "roofline": {
            "kernel": dom,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "bytes_per_launch": dom_bytes,
        },
        "cpu_baseline": None,
    }
    # the rate against what this GPU moves in a plain 1 GiB device-to-device
    # copy (read + write bytes), beside the published peak
    cb, cms = time_copy(1024)
    copy_gbs = 2 * cb / (cms * 1e-3) / 1e9
    line["copy_gbs"] = round(copy_gbs, 1)
    line["pct_of_copy"] = round(100.0 * gbs / copy_gbs, 2)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(dtype_name, batch, dim, seqlen, dstate)
        line["cpu_baseline"]["gpu_speedup"] = round(gbs / line["cpu_baseline"]["value"], 1)
        # the PyTorch oracle beside it, on a bounded sample
        line["cpu_baseline"]["selective_scan_ref"] = cpu_ref_sample(dtype_name, min(seqlen, 2048), dstate)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
