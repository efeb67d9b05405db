"""Benchmark of the MI355X MoE feed-forward (MXFP4 experts) on one GPU.

Default workload: GPT-OSS-20B-shaped MoE layer, decode (T=8 tokens, D=F=2880, E=32, top-4, bf16
activations, MXFP4 expert weights, seeded synthetic data).  One step = one full layer forward
(RmsNorm -> router -> top-k/softmax -> dispatch -> gate_up+SwiGLU -> down -> combine + residual)
with inputs already resident in HBM.  Four device copies of the layer are rotated so that the
256 MB Infinity Cache cannot serve a step's ~280 MB of expert weights from the previous step.

Prints ONE JSON line (rank 0): metric/value/unit plus a `roofline` object for the dominant kernel
(algorithmic bytes / FLOPs from the realised routing, divided by that kernel's average duration
measured with HIP events on the launch stream) and a `cpu_baseline` object (the CPU restatement
of the reference algorithm, timed on a bounded sample of the same workload on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "burn-extended_amd"))

METRIC = "MoE-layer tokens/s + HBM GB/s (decode) / FP4 MFMA util (prefill), 1 MI355X"
HBM_PEAK_GBS = 8000.0
FP4_PEAK_TFLOPS = 10100.0

WORKLOADS = {
    "20b_decode": dict(D=2880, F=2880, E=32, K=4, T=8, zipf=False),
    "20b_prefill": dict(D=2880, F=2880, E=32, K=4, T=4096, zipf=True),
    "120b_t1": dict(D=2880, F=2880, E=128, K=4, T=1, zipf=False),
    "120b_t64": dict(D=2880, F=2880, E=128, K=4, T=64, zipf=False),
    "120b_t8192": dict(D=2880, F=2880, E=128, K=4, T=8192, zipf=False),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="20b_decode", choices=sorted(WORKLOADS))
    ap.add_argument("--copies", type=int, default=4, help="device copies of the layer rotated per step")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (HBM counter calibration)")
    return ap.parse_args()


def copy_probe(mib):
    """A plain device-to-device copy of known size: under `rocprofv3 --pmc FETCH_SIZE` /
    `WRITE_SIZE` its per-dispatch counter values give the factor that turns those counters into
    HBM bytes on this GPU."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}), flush=True)


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (one MI355X per run); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from burnext_amd import moe, synth

    wl = WORKLOADS[args.workload]
    D, F, E, K, T = wl["D"], wl["F"], wl["E"], wl["K"], wl["T"]
    dev = 0
    torch.cuda.set_device(dev)
    bias = synth.zipf_router_bias(E, 1.1, gamma=1.0, seed=0) if wl["zipf"] else None
    data = synth.make_layer(D, F, E, K, seed=0, dtype="bf16", router_bias=bias)
    layers = []
    for i in range(max(1, args.copies)):
        layers.append(moe.MoeLayer(data, device=dev))
        print(f"[bench] layer copy {i + 1}/{max(1, args.copies)} resident", file=sys.stderr, flush=True)
    x_np = synth.make_tokens(T, D, seed=0, dtype="bf16")
    x = moe.to_device_x(x_np, "bf16", dev)
    y = torch.empty_like(x)
    ws = layers[0].workspace(T)

    # realised routing -> touched experts and segment sizes
    idx, _, _ = layers[0].route(x)
    idx_np = idx.cpu().numpy()
    counts = np.bincount(idx_np.ravel(), minlength=E)
    touched = int(np.count_nonzero(counts))

    def step(i):
        layers[i % len(layers)].forward(x, out=y, workspace=ws)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    ms_total = start.elapsed_time(end)
    ms_step = ms_total / args.steps

    # per-kernel durations: HIP event pairs recorded by the library around each launch on the
    # launch stream, over a second pass of the same steps
    for L in layers:
        L.profile_enable(True)
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    kern = {}
    for L in layers:
        L.profile_enable(False)
        for name, (ms, cnt) in L.profile_read().items():
            a = kern.setdefault(name, [0.0, 0])
            a[0] += ms
            a[1] += cnt
    kavg_us = {k: (v[0] / v[1] * 1e3) for k, v in kern.items() if v[1]}

    # algorithmic bytes per launch (realised routing; bf16 biases/router/activations)
    nk = T * K
    w1_bytes = 2 * F * ((D + 1) // 2) + 2 * F * ((D + 31) // 32) + 2 * F * 2
    w2_bytes = D * ((F + 1) // 2) + D * ((F + 31) // 32)
    kbytes = {
        "gate_up": touched * w1_bytes + T * D * 2 + nk * F * 4,
        "down": touched * w2_bytes + nk * F * 4 + nk * D * 4,
        "router": E * D * 2 + E * 2 + T * D * 2 + T * D * 2 + T * E * 4,
        "combine": nk * D * 4 + touched * D * 2 + 2 * T * D * 2 + nk * 12,
    }
    kflops = {"gate_up": 2 * nk * 2 * F * D, "down": 2 * nk * D * F}
    layer_bytes = synth.decode_bytes(data, touched, T, 2)
    dominant = max(kavg_us, key=kavg_us.get)
    traffic = measured_traffic(args.workload, dominant)
    if T >= 1024:
        fl = kflops.get(dominant, 0)
        ach = fl / (kavg_us[dominant] * 1e-6) / 1e12
        roof = {"bound": "mfma", "kernel": dominant, "achieved": round(ach, 2), "peak": FP4_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / FP4_PEAK_TFLOPS, 4), "traffic": traffic,
                "algorithmic_flops_per_launch": fl, "avg_launch_us": round(kavg_us[dominant], 2)}
    else:
        b = kbytes.get(dominant, 0)
        ach = b / (kavg_us[dominant] * 1e-6) / 1e9
        roof = {"bound": "hbm", "kernel": dominant, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes_per_launch": b,
                "avg_launch_us": round(kavg_us[dominant], 2)}

    out = {
        "metric": METRIC,
        "value": round(T / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 activations, MXFP4 weights with random e2m1 codes and e8m0 "
                "scales 119..123, random-init router/biases)",
        "config": {"workload": f"gpt-oss-20b MoE layer {args.workload}" if E == 32 else f"gpt-oss-120b MoE layer {args.workload}",
                   "tokens": T, "d_model": D, "ffn_hidden": F, "experts": E, "top_k": K,
                   "weights": "mxfp4 (e2m1 + e8m0 per 32)", "activations": "bf16", "gate_up_layout": "interleaved",
                   "layer_copies_rotated": len(layers), "touched_experts": touched,
                   "max_segment": int(counts.max())},
        "layer_hbm_gbs": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
        "layer_hbm_frac": round(layer_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "layer_algorithmic_bytes": layer_bytes,
        "kernels_avg_us": {k: round(v, 2) for k, v in kavg_us.items()},
        "roofline": roof,
    }
    if T >= 1024:
        fl = 6 * T * K * F * D
        out["layer_fp4_mfma_util"] = round(fl / (ms_step * 1e-3) / 1e12 / FP4_PEAK_TFLOPS, 4)

    print(f"[bench] timed {args.steps} steps: {ms_step * 1e3:.1f} us/step", file=sys.stderr, flush=True)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(data, x_np, args.cpu_seconds)
    for L in layers:
        L.close()
    print(json.dumps(out), flush=True)


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary
    (profiles/hbm_traffic_<workload>.txt: FETCH_SIZE and WRITE_SIZE per dispatch, scaled by a plain
    copy's counter readings); None when no summary covers it."""
    path = ROOT / "profiles" / f"hbm_traffic_{workload}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        f = line.split()
        if len(f) >= 3 and f[0] == "traffic" and f[1] == workload and f[2] == kernel:
            kv = dict(x.split("=", 1) for x in f[3:] if "=" in x)
            return int(float(kv["bytes"])) if "bytes" in kv else None
    return None


def cpu_baseline(data, x_np, budget_s):
    """Reference algorithm restated on the CPU (oracle/moe_oracle.c, literal loop structure of
    src/moe/mod.rs:129-411 with b2 added once), OpenMP over the host cores, on whole layer
    forwards of the same tokens until the time budget is spent."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    O.lib()
    T = x_np.shape[0]
    rows = x_np if T <= 256 else x_np[:256]
    n_fwd, t0 = 0, time.perf_counter()
    while True:
        O.moe_forward_reference(data, rows, b2_per_ftile=False)
        n_fwd += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n_fwd >= 50:
            break
    return {"value": round(n_fwd * rows.shape[0] / el, 2), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port",
            "sample": f"{n_fwd} layer forward(s) of {rows.shape[0]} tokens of this workload in {el:.1f} s "
                      f"(reference algorithm restated in C, f32, dense W1 per used expert)",
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
