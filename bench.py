"""Benchmark of the MI355X MoE feed-forward (MXFP4 experts) on one GPU.

Headline workload: GPT-OSS-20B-shaped MoE layer, decode (C2: T=8 tokens, D=F=2880, E=32, top-4,
bf16 activations, MXFP4 expert weights, seeded synthetic data).  One step = one full layer forward
(RmsNorm -> router -> top-k/softmax -> dispatch -> gate_up+SwiGLU -> down -> combine + residual)
with inputs already resident in HBM.  Several device copies of the layer are rotated so that the
256 MB Infinity Cache cannot serve a step's expert weights from the previous step.

The same run also measures the metric's prefill half (C3: T=4096 with the calibrated Zipf router
bias) as the `prefill` object, the GPT-OSS-120B-shaped layer (C4: E=128) at T = 1, 64 and 8192
as `sweep_120b`, and the full GPT-OSS-20B-shaped decoder decode (C5: 24 layers, batch 8, an
8192-row KV cache held full, greedy) as `decoder`.  `--workload NAME` measures one workload alone
(profiling runs).

Prints ONE JSON line: metric/value/unit plus, per workload, a `roofline` object for the dominant
kernel (algorithmic bytes or FLOPs from the realised routing, divided by that kernel's average
execution time: HIP events bound to each kernel dispatch, the kernel's own begin/end timestamps as
rocprofv3's kernel trace reports them) and a `cpu_baseline` object (the CPU restatement of the
reference algorithm, timed on a bounded sample of the same workload on the host cores).
"""
from __future__ import annotations

import argparse
import dataclasses
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
ZIPF_S = 1.1

WORKLOADS = {
    "20b_decode": dict(D=2880, F=2880, E=32, K=4, T=8, zipf=False, copies=4),
    "20b_prefill": dict(D=2880, F=2880, E=32, K=4, T=4096, zipf=True, copies=4),
    "120b_t1": dict(D=2880, F=2880, E=128, K=4, T=1, zipf=False, copies=8),
    "120b_t64": dict(D=2880, F=2880, E=128, K=4, T=64, zipf=False, copies=4),
    "120b_t8192": dict(D=2880, F=2880, E=128, K=4, T=8192, zipf=False, copies=4),
}
TIMING = ("kernel dispatch begin/end (pooled fence-free HIP event pair bound to each dispatch by "
          "hipExtLaunchKernel; steps queued behind a GPU sleep so the kernels run back to back)")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=None, choices=sorted(WORKLOADS),
                    help="measure this workload alone (default: 20b_decode headline + prefill + 120B sweep)")
    ap.add_argument("--copies", type=int, default=0, help="device copies of the layer rotated per step (0: per workload)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of each CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-120b", action="store_true", help="skip the 120B sweep of the default run")
    ap.add_argument("--no-decoder", action="store_true", help="skip the full-decoder leg of the default run")
    ap.add_argument("--decoder-steps", type=int, default=50, help="timed decode steps of the decoder leg")
    ap.add_argument("--decoder-only", action="store_true", help="measure the full-decoder leg alone")
    ap.add_argument("--fused-experts", action="store_true",
                    help="forward with BURNEXT_FUSED_EXPERTS (the opt-in one-launch experts kernel of decode batches)")
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


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


_SLEEP_RATE = []


def sleep_cycles_per_s():
    """Rate of torch.cuda._sleep's cycle counter (a bounded spin kernel), measured once."""
    import torch
    if not _SLEEP_RATE:
        torch.cuda._sleep(1000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(2_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_RATE.append(2_000_000 / max(e0.elapsed_time(e1) * 1e-3, 1e-6))
    return _SLEEP_RATE[0]


def make_data(name):
    from burnext_amd import synth
    wl = WORKLOADS[name]
    bias = synth.zipf_router_bias(wl["E"], ZIPF_S, gamma=synth.ZIPF_GAMMA_C3, seed=0) if wl["zipf"] else None
    return synth.make_layer(wl["D"], wl["F"], wl["E"], wl["K"], seed=0, dtype="bf16", router_bias=bias)


def make_layers(data, copies, dev=0):
    from burnext_amd import moe
    layers = []
    for i in range(copies):
        layers.append(moe.MoeLayer(data, device=dev))
    log(f"{copies} device copies of the E={data.num_experts} layer resident")
    return layers


FORWARD_FLAGS = [3]  # BURNEXT_FORWARD_DEFAULT; | BURNEXT_FUSED_EXPERTS under --fused-experts


def measure(name, layers, data, steps, warmup, with_cpu, cpu_seconds):
    """Times `steps` layer forwards (after `warmup`) on resident inputs; returns the workload's
    figures: tokens/s, per-kernel execution times, the dominant kernel's roofline, routing."""
    import numpy as np
    import torch

    from burnext_amd import moe, synth

    wl = WORKLOADS[name]
    D, F, E, K, T = wl["D"], wl["F"], wl["E"], wl["K"], wl["T"]
    x_np = synth.make_tokens(T, D, seed=0, dtype="bf16")
    x = moe.to_device_x(x_np, "bf16", 0)
    y = torch.empty_like(x)
    ws = layers[0].workspace(T)

    # realised routing -> touched experts and segment sizes
    idx, _, _ = layers[0].route(x)
    idx_np = idx.cpu().numpy()
    counts = np.bincount(idx_np.ravel(), minlength=E)
    touched = int(np.count_nonzero(counts))

    flags = FORWARD_FLAGS[0]

    def step(i):
        layers[i % len(layers)].forward(x, out=y, workspace=ws, flags=flags)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / steps

    # per-kernel execution times over a second pass of the same steps.  A first recorded pass fills
    # each layer's pool of event pairs (read and discarded), so the measured pass creates no events
    # between its launches.  Timed launches cost the host more than plain ones; where that makes the
    # pass host-bound (short decode steps), its kernels would start on an idle GPU, so the measured
    # pass queues its steps in chunks behind a bounded GPU sleep longer than the chunk's enqueue
    # time and its kernels run back to back as in the untimed pass.  (Where the host keeps ahead,
    # the steps go out directly: queued behind a sleep, the prefill GEMMs measured 15% slower under
    # the kernel tracer too, so prefill-sized batches (whose steps are long next to any launch gap)
    # never queue behind one.)
    for L in layers:
        L.profile_enable(True)
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    host_s = (time.perf_counter() - t0) / steps
    torch.cuda.synchronize()
    for L in layers:
        L.profile_read()
    for L in layers:
        L.profile_enable(True)  # every pass read: its pairs return to the pool
    gated = host_s > ms_step * 1e-3 and T < 1024
    chunk = 20 if gated else steps
    spans = []  # GPU time of each chunk's steps (after its sleep): the measured pass's own step
    for c0 in range(0, steps, chunk):
        n = min(chunk, steps - c0)
        if gated:
            torch.cuda._sleep(int(2.0 * n * host_s * sleep_cycles_per_s()) + 10000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(c0, c0 + n):
            step(i)
        e1.record()
        spans.append((e0, e1))
    torch.cuda.synchronize()
    prof_step_us = sum(a.elapsed_time(b) for a, b in spans) * 1e3 / steps
    kern = {}
    for L in layers:
        L.profile_enable(False)
        for k, (ms, cnt) in L.profile_read().items():
            a = kern.setdefault(k, [0.0, 0])
            a[0] += ms
            a[1] += cnt
    kavg_us = {k: (v[0] / v[1] * 1e3) for k, v in kern.items() if v[1]}
    # every kernel of a step runs on one stream, one launch each: their exclusive intervals are
    # disjoint, so their sum cannot pass the step of the pass they were measured in (whose event
    # pairs cost a little over the untimed pass's step)
    ksum_us = sum(v[0] for v in kern.values()) * 1e3 / steps
    log(f"{name}: {ms_step * 1e3:.1f} us/step, kernels {', '.join(f'{k} {v:.1f}' for k, v in kavg_us.items())}, "
        f"sum {ksum_us:.1f} in a timed pass of {prof_step_us:.1f} us/step (its launches enqueue at "
        f"{host_s * 1e6:.1f} us per step{', queued behind a GPU sleep' if gated else ''})")
    if ksum_us > prof_step_us:
        log(f"{name}: WARNING kernel durations sum to {ksum_us:.1f} us, above the {prof_step_us:.1f} us step "
            f"of their pass")

    # algorithmic bytes / FLOPs per launch (realised routing; bf16 biases, router, activations)
    nk = T * K
    w1_bytes = 2 * F * ((D + 1) // 2) + 2 * F * ((D + 31) // 32) + 2 * F * 2
    w2_bytes = D * ((F + 1) // 2) + D * ((F + 31) // 32)
    kbytes = {
        "gate_up": touched * w1_bytes + T * D * 2 + nk * F * 4,
        "down": touched * w2_bytes + nk * F * 4 + nk * D * 4,
        "router": E * D * 2 + E * 2 + T * D * 2 + T * D * 2 + T * E * 4,
        "combine": nk * D * 4 + touched * D * 2 + 2 * T * D * 2 + nk * 12,
        # the fused decode experts: both projections' weights and biases, the token rows, one f32
        # output row per slot (its per-slice partial rows are not algorithmic)
        "experts": touched * (w1_bytes + w2_bytes + D * 2) + T * D * 2 + nk * D * 4,
    }
    kflops = {"gate_up": 2 * nk * 2 * F * D, "down": 2 * nk * D * F}
    layer_bytes = synth.decode_bytes(data, touched, T, 2)
    stage_us = dict(kavg_us)
    dominant = max((k for k in stage_us if k in kbytes), key=stage_us.get)
    label = dominant
    traffic = measured_traffic(name, dominant)
    prefill = T >= 1024
    if prefill:
        fl = kflops[dominant]
        ach = fl / (stage_us[dominant] * 1e-6) / 1e12
        roof = {"bound": "mfma", "kernel": label, "achieved": round(ach, 2), "peak": FP4_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / FP4_PEAK_TFLOPS, 4), "traffic": traffic,
                "algorithmic_flops_per_launch": fl, "avg_launch_us": round(stage_us[dominant], 2), "timing": TIMING}
    else:
        b = kbytes[dominant]
        ach = b / (stage_us[dominant] * 1e-6) / 1e9
        roof = {"bound": "hbm", "kernel": label, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes_per_launch": b,
                "avg_launch_us": round(stage_us[dominant], 2), "timing": TIMING}
    out = {
        "value": round(T / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms_step, 5),
        "config": {"workload": f"gpt-oss-{'20b' if E == 32 else '120b'} MoE layer {name}", "tokens": T, "d_model": D,
                   "ffn_hidden": F, "experts": E, "top_k": K, "weights": "mxfp4 (e2m1 + e8m0 per 32)",
                   "activations": "bf16", "gate_up_layout": "interleaved", "layer_copies_rotated": len(layers),
                   "touched_experts": touched, "max_segment": int(counts.max())},
        "layer_hbm_gbs": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
        "layer_hbm_frac": round(layer_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "layer_algorithmic_bytes": layer_bytes,
        "kernels_avg_us": {k: round(v, 2) for k, v in kavg_us.items()},
        "kernels_sum_us": round(ksum_us, 2),
        "kernels_pass_us_per_step": round(prof_step_us, 2),
        "roofline": roof,
    }
    if prefill:
        out["layer_fp4_mfma_util"] = round(6 * T * K * F * D / (ms_step * 1e-3) / 1e12 / FP4_PEAK_TFLOPS, 4)
    if wl["zipf"]:
        by_rank = synth.zipf_rank_counts_from_idx(idx_np, E, seed=0)
        out["config"]["router_bias"] = f"zipf s={ZIPF_S} gamma={synth.ZIPF_GAMMA_C3} (calibrated)"
        out["segment_histogram_by_zipf_rank"] = by_rank.tolist()
        out["segment_ideal_by_zipf_rank"] = [int(round(v)) for v in synth.zipf_ideal_counts(E, ZIPF_S, T, K)]
    if flags & 4:
        out["config"]["experts"] = "fused (BURNEXT_FUSED_EXPERTS)"
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(data, x_np, cpu_seconds)
    return out


def measure_decoder(steps, warmup, with_cpu, kv_bf16_leg=True):
    """C5: the GPT-OSS-20B-shaped decoder (24 layers, d_model 2880, 64 q / 8 kv heads of 64,
    alternating 128-row window and full layers with learned sinks, YaRN factor 32 base 150000,
    vocabulary 201088, 32 experts top-4 per MoE layer) decoding batch 8 greedily with its
    8192-row f32 KV cache held full (loaded with 8191 rows, so every timed step attends over 8192
    rows in the full layers and evicts the oldest).  One step = one token per batch row through
    all 24 layers, final norm, LM head and argmax."""
    import numpy as np
    import torch

    from burnext_amd import decoder as DEC

    B, pre = 8, 8191
    cfg = DEC.GptOssConfig(max_seq_len=pre + warmup + steps + 64)
    t0 = time.perf_counter()
    data = DEC.make_decoder(cfg, seed=0, sinks_std=0.5)
    log(f"decoder: weights generated in {time.perf_counter() - t0:.1f} s")
    dev = DEC.GptOssDecoder(data, max_batch=B)
    shape = (cfg.n_layers, B, pre, cfg.kv_heads, cfg.head_dim)
    g = torch.Generator(device="cuda:0").manual_seed(0)
    k = torch.randn(shape, generator=g, device="cuda:0") * 0.6
    v = torch.randn(shape, generator=g, device="cuda:0")
    dev.cache_load(k, v)
    torch.cuda.synchronize()
    del k, v
    tok = torch.from_numpy(np.arange(B, dtype=np.int32) * 1009 % cfg.vocab_size).cuda()
    ws = dev.workspace(B)
    pos = pre
    for _ in range(warmup):
        tok = dev.decode(tok, pos, workspace=ws)
        pos += 1
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        tok = dev.decode(tok, pos, workspace=ws)
        pos += 1
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # algorithmic HBM bytes of one step: dense weights (bf16) and their f32 biases / norms, the
    # touched experts of every MoE layer (expected count under uniform routing), the cache rows
    # each layer attends over (k and v, f32) and the new rows, the LM head
    D, L, V = cfg.d_model, cfg.n_layers, cfg.vocab_size
    qd, kd = cfg.n_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    touched = cfg.num_experts * (1 - (1 - cfg.experts_per_token / cfg.num_experts) ** B)
    m = data.moe[0]
    moe_b = touched * m.expert_bytes() + cfg.num_experts * D * 2 + cfg.num_experts * 2 + 2 * B * D * 4
    dense_b = ((qd + 2 * kd) * D + D * qd) * 2 + (qd + 2 * kd + D + D) * 4 + cfg.n_heads * 4
    rows = sum(min(cfg.layer_window(l) or cfg.cache_len, cfg.cache_len) for l in range(L))
    kv_b = rows * B * kd * 4 * 2 + L * B * kd * 4 * 2
    step_b = L * (dense_b + moe_b) + kv_b + V * D * 2 + D * 4 + B * D * 2
    out = {"value": round(B / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
           "config": {"workload": "gpt-oss-20b decoder decode (C5)", "layers": L, "batch": B, "d_model": D,
                      "heads": cfg.n_heads, "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
                      "window": f"every other layer {cfg.window} rows (full on even)", "sinks": "learned",
                      "rope": f"yarn factor {cfg.rope_scaling_factor} base {cfg.rope_theta}",
                      "kv_cache": f"{cfg.cache_len} rows f32, held full (rolling)", "vocab": V,
                      "experts": cfg.num_experts, "top_k": cfg.experts_per_token, "sampling": "greedy",
                      "data": "random-init weights (seed 0), random cache rows, greedy-fed tokens"},
           "step_algorithmic_bytes": int(step_b),
           "step_hbm_gbs": round(step_b / (ms * 1e-3) / 1e9, 1),
           "step_hbm_frac": round(step_b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "step_bytes_note": f"expected touched experts {touched:.1f} of {cfg.num_experts} per layer under "
                              f"uniform routing; cache rows attended per step summed over layers: {rows}"}
    log(f"decoder: {ms:.3f} ms/step, {out['value']} tokens/s, step {out['step_hbm_gbs']} GB/s")
    if kv_bf16_leg:
        # options beyond the reference, on second model objects over the same MoE layers: bf16 cache
        # rows (half the attention bytes), the expert projections on bf16-rounded rows (one MFMA
        # term), and both; parity bar 2e-2 for each instead of the f32 decoder's 5e-4
        kv_b_all = rows * B * kd * 4 * 2 + L * B * kd * 4 * 2

        def leg(key, note, **changes):
            nonlocal dev, tok
            cfgx = dataclasses.replace(cfg, **changes)
            datax = dataclasses.replace(data, cfg=cfgx)
            moe_layers = dev.moe_layers
            dev.close()
            dev = DEC.GptOssDecoder(datax, max_batch=B, moe_layers=moe_layers)
            k = torch.randn(shape, generator=g, device="cuda:0") * 0.6
            v = torch.randn(shape, generator=g, device="cuda:0")
            dev.cache_load(k, v)
            torch.cuda.synchronize()
            del k, v
            wsx = dev.workspace(B)
            p = pre
            for _ in range(warmup):
                tok = dev.decode(tok, p, workspace=wsx)
                p += 1
            torch.cuda.synchronize()
            start.record()
            for _ in range(steps):
                tok = dev.decode(tok, p, workspace=wsx)
                p += 1
            end.record()
            torch.cuda.synchronize()
            msx = start.elapsed_time(end) / steps
            stepx = step_b - (kv_b_all / 2 if changes.get("kv_bf16") else 0)
            out[key] = {"value": round(B / (msx * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(msx, 4),
                        "step_hbm_frac": round(stepx / (msx * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "note": note}
            log(f"decoder ({note}): {msx:.3f} ms/step, {out[key]['value']} tokens/s")

        leg("kv_bf16", "bf16 cache rows (the reference keeps f32)", kv_bf16=True)
        leg("experts_bf16", "expert projections on bf16-rounded rows (the reference's are f32)", experts_bf16=True)
        leg("kv_bf16_experts_bf16", "bf16 cache rows and bf16 expert rows", kv_bf16=True, experts_bf16=True)
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline_decoder(data, B, pre)
    dev.close()
    return out


def cpu_baseline_decoder(data, B, pre):
    """One decode step of the same decoder on the host cores: the CPU restatement of the
    reference's decode (oracle/decoder_oracle.c: dense Linear, RoPE, cache roll, sink attention,
    the MoE layer by oracle/moe_oracle.c), f32, with the same 8191 cached rows per layer."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    O.lib()
    orc = O.DecoderOracle(data, B)
    rng = np.random.default_rng(0)
    for l in range(data.cfg.n_layers):  # cache contents do not change the work
        orc.k[l, :, :pre] = rng.standard_normal((B, pre, data.cfg.kv_heads, data.cfg.head_dim), np.float32) * 0.6
        orc.v[l, :, :pre] = rng.standard_normal((B, pre, data.cfg.kv_heads, data.cfg.head_dim), np.float32)
    orc.used = pre
    tok = (np.arange(B, dtype=np.int32) * 1009) % data.cfg.vocab_size
    t0 = time.perf_counter()
    orc.step(tok, pre)
    el = time.perf_counter() - t0
    return {"value": round(B / el, 3), "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"1 decode step (batch {B}, 24 layers, 8192-row cache) in {el:.1f} s "
                      "(reference decode restated in C, f32)", "cpu": _cpu_model()}


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
    forwards of the same tokens (the first 256 of a larger batch) until the time budget is spent."""
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
    what = f"{rows.shape[0]} tokens" if T <= 256 else f"the first {rows.shape[0]} of the {T} tokens"
    return {"value": round(n_fwd * rows.shape[0] / el, 2), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port",
            "sample": f"{n_fwd} layer forward(s) of {what} of this workload in {el:.1f} s "
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


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (one MI355X per run); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.fused_experts:
        FORWARD_FLAGS[0] = 3 | 4
    import torch

    torch.cuda.set_device(0)
    if args.decoder_only:
        res = measure_decoder(args.decoder_steps, 5, not args.no_cpu)
        print(json.dumps({"decoder": res}), flush=True)
        return
    head = args.workload or "20b_decode"
    data = make_data(head)
    layers = make_layers(data, args.copies or WORKLOADS[head]["copies"])
    res = measure(head, layers, data, args.steps, args.warmup, not args.no_cpu, args.cpu_seconds)
    for L in layers:
        L.close()
    del layers
    out = {"metric": METRIC, "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded N(0,1) bf16 activations, MXFP4 weights with random e2m1 codes and e8m0 "
                   "scales 119..123, random-init router/biases)"}
    out.update(res)
    if args.workload is None:
        # the metric's prefill half (C3), same run
        pdata = make_data("20b_prefill")
        layers = make_layers(pdata, WORKLOADS["20b_prefill"]["copies"])
        out["prefill"] = measure("20b_prefill", layers, pdata, args.steps, args.warmup, not args.no_cpu,
                                 args.cpu_seconds)
        for L in layers:
            L.close()
        del layers
        if not args.no_120b:
            # 120B (C4): one set of layer copies serves the three batch sizes
            bdata = make_data("120b_t64")
            layers = make_layers(bdata, WORKLOADS["120b_t1"]["copies"])
            sweep = {}
            for name in ("120b_t1", "120b_t64", "120b_t8192"):
                use = layers[:WORKLOADS[name]["copies"]]
                r = measure(name, use, bdata, args.steps, args.warmup, False, 0)
                sweep[name.split("_")[1]] = {k: r[k] for k in ("value", "unit", "ms_per_step", "layer_hbm_frac",
                                                                "layer_fp4_mfma_util", "kernels_avg_us",
                                                                "kernels_sum_us", "kernels_pass_us_per_step", "roofline", "config") if k in r}
            out["sweep_120b"] = sweep
            for L in layers:
                L.close()
            del layers
        if not args.no_decoder:
            out["decoder"] = measure_decoder(args.decoder_steps, 5, not args.no_cpu)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
