"""Selective-scan fwd+bwd benchmark on one MI355X.

Workload (default): selective_scan_fn forward + backward, fp32, batch 8,
dim 1536 (Mamba-130m d_inner), dstate 16, seqlen 2048, variable B/C (one
group), z gate, D skip, delta_bias with softplus; dout ~ N(0,1).  A step is
one forward + backward over that batch with all inputs already in HBM.

Prints one JSON line.  ``value`` is the algorithmic HBM bytes of one
forward + backward (inputs read and outputs written once, no checkpoints or
scratch) divided by the measured time per step, in GB/s.  ``roofline``
describes the dominant kernel, timed with HIP events on the stream it runs
on; ``cpu_baseline`` times the CPU oracle (pure-PyTorch selective_scan_ref)
on a bounded slice of the same workload on this host's cores.

``--calibrate-copy MIB`` instead times a plain device-to-device copy of MIB
MiB (torch's copy kernel); under ``rocprofv3 --pmc FETCH_SIZE`` /
``WRITE_SIZE`` it gives the factor between those counters and bytes actually
read / written, which scales the scan kernels' counters into ``traffic``.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload NAME] [--no-cpu]
       python bench.py --calibrate-copy 1024
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
}
DEFAULT = "ss_fwd_bwd_b8_d1536_n16_l2048_f32"


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


def cpu_baseline(dtype_name, seqlen, dstate, min_seconds=10.0, max_dim=1536):
    """Times the CPU oracle (fwd + autograd bwd) on 1 batch row x `d` channels
    at the full sequence length, on this host's cores.  `d` starts at 192 and
    is doubled until one run takes at least `min_seconds` (bounded by
    `max_dim`), so the sample is a few seconds to a few tens of seconds."""
    import torch
    from oracle.selective_scan_ref import make_inputs, selective_scan_ref
    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    b, d = 1, 192
    while True:
        x = make_inputs(b, d, dstate, seqlen, seed=1001, dtype=getattr(torch, dtype_name))
        ins = {k: x[k].clone().requires_grad_(True) for k in names}
        t0 = time.perf_counter()
        out = selective_scan_ref(ins["u"], ins["delta"], ins["A"], ins["B"], ins["C"], ins["D"],
                                 z=ins["z"], delta_bias=ins["delta_bias"], delta_softplus=True)
        out.backward(x["dout"])
        dt = time.perf_counter() - t0
        print(f"[bench] cpu oracle batch {b} x dim {d}: {dt:.2f} s", file=sys.stderr, flush=True)
        if dt >= min_seconds or d * 2 > max_dim:
            break
        d *= 2
    s = 2 if dtype_name != "float32" else 4
    fwd_b, bwd_b = algorithmic_bytes(b, d, dstate, seqlen, s)
    return {
        "value": round((fwd_b + bwd_b) / dt / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"selective_scan_ref (pure PyTorch) fwd+bwd on batch {b} x dim {d} x seqlen {seqlen} "
                  f"x dstate {dstate} ({dtype_name}), one run of {dt:.2f} s; same byte formula as value",
        "elems_per_s": round(b * d * seqlen / dt, 1),
        "seconds": round(dt, 3),
    }


def calibrate_copy(mib, reps=5):
    """Copies `mib` MiB device to device `reps` times; prints one JSON line."""
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
    nbytes = n * 4
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "ms": round(ms, 5),
                      "GB/s (read + write)": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only time a plain device copy of MIB MiB (counter calibration)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the selective scan would shard by batch or channel "
              "(see DESIGN.md), which is not built here.", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return

    import torch
    from mamba_amd import selective_scan as ss
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    from oracle.selective_scan_ref import make_inputs  # seeded synthetic inputs only

    batch, dim, dstate, seqlen, dtype_name, seed = WORKLOADS[args.workload]
    dtype = getattr(torch, dtype_name)
    s = 2 if dtype != torch.float32 else 4
    dev = torch.device("cuda:0")
    x = make_inputs(batch, dim, dstate, seqlen, seed=seed, dtype=dtype)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    g = {k: x[k].to(dev).requires_grad_(True) for k in names}
    dout = x["dout"].to(dev)
    params = [g[k] for k in names]

    def step():
        out = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                delta_bias=g["delta_bias"], delta_softplus=True)
        return torch.autograd.grad(out, params, dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
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
        if ws > 0:   # the backward is three launches: clear slices and accumulators, scan, sum slices
            bname = f"ss_zero_segs + {bname} + ss_ws_reduce"
        kernel_ms = {}
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

    traffic = None
    tpath = os.path.join(_HERE, "profiles", f"traffic_{args.workload}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dom)

    line = {
        "metric": "selective-scan fwd+bwd GB/s (% HBM peak) + elems/s, D=1536 N=16 L=2048",
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
            "bytes_per_launch": dom_bytes,
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(dtype_name, seqlen, dstate)
        line["cpu_baseline"]["gpu_speedup"] = round(gbs / line["cpu_baseline"]["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
