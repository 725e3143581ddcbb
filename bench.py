"""Benchmark: one Qwen-Image-shaped 60-block MMDiT denoiser step at 1024x1344
(5376 image + 256 text tokens, hidden 3072, 24 x 128 heads, MLP 12288) on one
MI355X, bf16 compute (or int8 block-quantised weights with --int8), inputs
resident in HBM before the timed region.

Prints one JSON line: s/step, the roofline of the dominant kernel (algorithmic
flops per launch over its HIP-event-timed average launch), and the CPU
baseline (the oracle's restatement of the reference's C# CPU layer path,
timed on this host over one block of the same step and scaled to 60 blocks).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--int8] [--no-cpu-baseline]
    python bench.py --calibrate-copy    # a plain 1 GiB device copy, for scaling HBM counters

The roofline's `traffic` (HBM bytes per launch of the dominant kernel) is
read from the committed rocprofv3 counter summary for that kernel under
profiles/ (a `bytes_per_launch:` line), null when there is none.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (and fp16)
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def calibrate_copy(reps=5):
    """A plain copy kernel of known size: the library's elementwise identity
    over a 1 GiB bf16 tensor (reads 1 GiB, writes 1 GiB per launch). The
    FETCH_SIZE and WRITE_SIZE counters of these launches give the factor
    that turns those counters into bytes."""
    import naivediffusion_amd as nd
    from naivediffusion_amd.graph import Ops
    from naivediffusion_amd.tensors import HostDataType as DT

    dev = nd.Device()
    shape = [1, 1, 16384, 32768]
    g = nd.Graph(dev)
    x = g.Input(DT.BFloat16, shape)
    model = nd.CompiledModel(g, [Ops.Identity(x)], dev)
    src = dev.Normal(DT.BFloat16, shape, 1)
    dst = dev.Empty(DT.BFloat16, shape)
    for _ in range(reps):
        model.DispatchInto([src], [dst])
    dev.Synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read_per_launch": 2 << 29, "bytes_written_per_launch": 2 << 29,
                      "launches": reps}), flush=True)


def read_traffic(kernel):
    """HBM bytes per launch of `kernel` from its committed counter summary."""
    for path in sorted((ROOT / "profiles").glob(f"{kernel}_*traffic*.md")):
        for line in path.read_text().splitlines():
            if line.strip().startswith("bytes_per_launch:"):
                return float(line.split(":", 1)[1].split()[0]), path.name
    return None, None


def cpu_baseline(device, cfg, seed, ni, nt):
    """The oracle (the C restatement of the reference's CpuMath layer path,
    fp32, OpenMP) on one block of the same step, scaled to cfg.blocks."""
    import oracle
    from naivediffusion_amd import mmdit, rng
    from naivediffusion_amd.tensors import HostDataType as DT

    D = cfg.width
    names = list(mmdit.block_weight_shapes(cfg, 0))
    dev_w = mmdit.device_weights(device, cfg, seed, names)
    w = {k: t.Download().ToFloats() for k, t in dev_w.items()}
    for t in dev_w.values():
        t.Dispose()

    def stream(s):
        p = f"blocks.0.{s}"
        return dict(w_mod=w[f"{p}_mod.weight"], b_mod=w[f"{p}_mod.bias"], w_qkv=w[f"{p}_qkv.weight"],
                    b_qkv=w[f"{p}_qkv.bias"], norm_q=w[f"{p}_norm_q.weight"], norm_k=w[f"{p}_norm_k.weight"],
                    w_o=w[f"{p}_out.weight"], b_o=w[f"{p}_out.bias"], w_fc1=w[f"{p}_fc1.weight"],
                    b_fc1=w[f"{p}_fc1.bias"], w_fc2=w[f"{p}_fc2.weight"], b_fc2=w[f"{p}_fc2.bias"])

    xi = device.Normal(DT.Float32, [ni, D], rng.tensor_seed(seed, "cpu.x_img")).Download().ToFloats()
    xt = device.Normal(DT.Float32, [nt, D], rng.tensor_seed(seed, "cpu.x_txt")).Download().ToFloats()
    temb = device.Normal(DT.Float32, [D], rng.tensor_seed(seed, "cpu.temb")).Download().ToFloats()
    cos, sin = mmdit.rope_tables(64, 84, nt)
    oracle.lib()
    threads = len(os.sched_getaffinity(0))
    log(f"cpu baseline: one block on the oracle, {threads} threads")
    t0 = time.perf_counter()
    oracle.mmdit_block(xi, xt, temb, stream("img"), stream("txt"), cfg.heads, cos, sin)
    dt = time.perf_counter() - t0
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": dt * cfg.blocks,
        "unit": "s/step",
        "cores": threads,
        "kind": "port",
        "sample": (f"one MMDiT block ({ni} image + {nt} text tokens, hidden {D}, fp32) on the oracle's C restatement "
                   f"of the reference CpuMath layer path in {dt:.2f} s, x{cfg.blocks} blocks (extrapolated); "
                   f"host CPU: {cpu_model}"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--int8", action="store_true", help="int8 block-quantised weights (bf16 compute)")
    ap.add_argument("--blocks", type=int, default=60)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true", help="run only the 1 GiB copy used to scale counters")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} (WORLD_SIZE {world}) is not supported; "
              "the multi-GPU sharding of this path is a design note, not a build.", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return

    import naivediffusion_amd as nd
    from naivediffusion_amd import mmdit, rng
    from naivediffusion_amd.tensors import HostDataType as DT, HostTensor

    cfg = mmdit.MmditConfig(blocks=args.blocks)
    lat_h, lat_w, nt = 128, 168, 256
    ni = (lat_h // cfg.patch) * (lat_w // cfg.patch)
    seed = 20261201
    dev = nd.Device()
    log(f"device {dev.AdapterName}")

    t0 = time.perf_counter()
    weights = mmdit.device_weights(dev, cfg, seed)
    log(f"synthetic weights on the device in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    model = mmdit.build_step_model(dev, cfg, weights, 1, nt, lat_h, lat_w, DT.BFloat16, args.int8)
    compiled = model.Compiled
    log(f"graph built and compiled in {time.perf_counter() - t0:.1f} s: {compiled.KernelCount} kernels/step, "
        f"{compiled.PersistentSize / 1e9:.1f} GB weights, {compiled.TemporarySize / 1e9:.2f} GB scratch")

    n = ni + nt
    cos, sin = mmdit.rope_tables(lat_h // cfg.patch, lat_w // cfg.patch, nt)
    inputs = [
        dev.Normal(DT.Float32, [1, cfg.latent_channels, lat_h, lat_w], rng.tensor_seed(seed, "latent")),
        dev.Normal(DT.Float32, [1, 1, nt, cfg.text_dim], rng.tensor_seed(seed, "text")),
        dev.Upload(HostTensor.FromFloats(mmdit.time_embedding(0.5, cfg.time_dim).reshape(1, 1, 1, cfg.time_dim))),
        dev.Upload(HostTensor.FromFloats(cos.reshape(1, n, 1, 64))),
        dev.Upload(HostTensor.FromFloats(sin.reshape(1, n, 1, 64))),
    ]
    out = [dev.Empty(DT.Float32, [1, cfg.latent_channels, lat_h, lat_w])]

    for i in range(args.warmup):
        compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    log(f"warmup done ({args.warmup} steps)")

    # Timed region: every kernel bracketed by HIP events on the device's
    # stream (the stream all kernels are launched on).
    compiled.SetProfiling(True)
    dev.Synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    elapsed = time.perf_counter() - t0
    prof = compiled.Profile()
    compiled.SetProfiling(False)
    s_per_step = elapsed / args.steps
    log(f"{args.steps} steps in {elapsed:.3f} s: {s_per_step * 1e3:.1f} ms/step")

    total_flops = sum(e["flops"] for e in prof.values()) / args.steps
    kernel_ms = sum(e["ms"] for e in prof.values()) / args.steps
    for name, e in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
        tf = e["flops"] / (e["ms"] * 1e-3) / 1e12 if e["ms"] else 0.0
        gbs = e["bytes"] / (e["ms"] * 1e-3) / 1e9 if e["ms"] else 0.0
        log(f"  {name:28s} {e['launches'] // args.steps:5d}/step {e['ms'] / args.steps:9.2f} ms/step "
            f"{tf:8.1f} TFLOP/s {gbs:8.1f} GB/s")
    gemm = {k: v for k, v in prof.items() if k.startswith("gemm_") and "generic" not in k}
    dom_name, dom = max(gemm.items(), key=lambda kv: kv[1]["ms"])
    per_launch_flops = dom["flops"] / dom["launches"]
    avg_ms = dom["ms"] / dom["launches"]
    achieved = per_launch_flops / (avg_ms * 1e-3) / 1e12
    traffic, traffic_src = read_traffic(dom_name)

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(dev, cfg, seed, ni, nt)
            log(f"cpu baseline {cpu['value']:.1f} s/step ({cpu['cores']} threads)")
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline failed: {e!r}")

    result = {
        "metric": "Qwen-Image DiT s/step @1024x1344 (bf16/int8 wts), 1 MI355X; % MFMA peak",
        "value": s_per_step,
        "unit": "s/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": s_per_step * 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) latent and text, N(0,0.02) bf16 weights made on the GPU)",
        "config": {
            "workload": (f"Qwen-Image-shaped MMDiT denoiser step, {cfg.blocks} dual-stream blocks, 1024x1344 "
                         f"(latent 16x{lat_h}x{lat_w}, 2x2 patch: {ni} image + {nt} text tokens), hidden 3072, "
                         f"24x128 heads, MLP 12288, batch 1, "
                         + ("int8 block-32 weights" if args.int8 else "bf16 weights")),
            "blocks": cfg.blocks,
            "image_tokens": ni,
            "text_tokens": nt,
            "weights": "int8" if args.int8 else "bf16",
            "algorithmic_tflop_per_step": total_flops / 1e12,
            "achieved_tflops_step": total_flops / s_per_step / 1e12,
            "step_frac_of_mfma_peak": total_flops / s_per_step / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "kernel_ms_per_step": kernel_ms,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": dom_name,
            "achieved": achieved,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
            "traffic": traffic,
            "traffic_unit": "bytes/launch",
            "traffic_source": traffic_src,
            "algorithmic_flop_per_launch": per_launch_flops,
            "launches_per_step": dom["launches"] // args.steps,
            "avg_launch_ms": avg_ms,
        },
        "kernels": {k: {"ms_per_step": v["ms"] / args.steps, "launches_per_step": v["launches"] // args.steps,
                        "tflops": (v["flops"] / (v["ms"] * 1e-3) / 1e12) if v["ms"] else 0.0,
                        "gbs": (v["bytes"] / (v["ms"] * 1e-3) / 1e9) if v["ms"] else 0.0}
                    for k, v in prof.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
