"""Benchmark: one Qwen-Image-shaped 60-block MMDiT denoiser step at 1024x1344
(5376 image + 256 text tokens, hidden 3072, 24 x 128 heads, MLP 12288) on one
MI355X, bf16 compute (or int8 block-quantised weights with --int8), inputs
resident in HBM before the timed region.

Prints one JSON line: s/step, the roofline of the dominant kernel (algorithmic
flops per launch over its average launch, timed by HIP events around its
launches inside the timed steps), and the CPU baseline (the oracle's
restatement of the reference's C# CPU layer path, timed on this host over one
block of the same step and scaled to 60 blocks). The per-family breakdown
comes from one untimed step with every kernel bracketed.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--int8] [--compute bf16|f32|f16] [--no-cpu-baseline] [--no-replay]
    python bench.py --workload anima|sdxl|qwen   # the Anima DiT / SDXL UNet / Qwen-Image 2.1 steps
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
# The per-family breakdown names the second stream's kernels apart
# ("...@lane1"): that stream's launches wait beside the first stream's work
# and are off the step's critical path, so summing them into one family with
# the first stream's would hide both rates.
os.environ.setdefault("NDX_PROFILE_LANES", "1")

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (and fp16)
FP32_PEAK_TFLOPS = 157.3         # MI355X fp32 matrix
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


def read_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` in `workload` from its committed
    counter summary (profiles/<kernel>_<workload>_..._traffic.md)."""
    for path in sorted((ROOT / "profiles").glob(f"{kernel}_{workload}_*traffic*.md")):
        for line in path.read_text().splitlines():
            if line.strip().startswith("bytes_per_launch:"):
                return float(line.split(":", 1)[1].split()[0]), path.name
    return None, None


def cpu_baseline(device, cfg, seed, ni, nt, grid=(64, 84), batch=1):
    """The oracle (the C restatement of the reference's CpuMath layer path,
    fp32, OpenMP) on one block of the same step (one batch element, a grid
    of image tokens), scaled to cfg.blocks x batch."""
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
    cos, sin = mmdit.rope_tables(grid[0], grid[1], nt)
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
    per = f" x{batch} batch elements" if batch > 1 else ""
    return {
        "value": dt * cfg.blocks * batch,
        "unit": "s/step",
        "cores": threads,
        "kind": "port",
        "sample": (f"one MMDiT block ({ni} image + {nt} text tokens, hidden {D}, fp32) on the oracle's C restatement "
                   f"of the reference CpuMath layer path in {dt:.2f} s, x{cfg.blocks} blocks{per} (extrapolated); "
                   f"host CPU: {cpu_model}"),
    }


def is_mfma_family(name):
    return (name.startswith("gemm_") and "generic" not in name) or name.startswith("conv_mfma") or \
        name.startswith("attention")


def measure(dev, compiled, inputs, out, steps, warmup):
    """W untimed steps; one untimed step with every kernel bracketed by HIP
    events (the per-family breakdown, and which MFMA family dominates); then
    K timed steps in which only that family's launches are bracketed, on the
    stream each is launched on, with nothing waiting between steps: the
    step time carries a few events per step instead of two per kernel and a
    wait per step. Returns (seconds per timed step, breakdown of the profiled
    step, the dominant family's events over the timed steps)."""
    for _ in range(warmup):
        compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    log(f"warmup done ({warmup} steps)")
    compiled.SetProfiling(True)
    compiled.DispatchInto(inputs, out)
    breakdown = compiled.Profile()
    compiled.SetProfiling(False)
    dominant = max((k for k in breakdown if is_mfma_family(k)), key=lambda k: breakdown[k]["ms"])
    compiled.SetProfiling(True, family=dominant)
    dev.Synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    elapsed = time.perf_counter() - t0
    timed = compiled.Profile()
    compiled.SetProfiling(False)
    log(f"{steps} steps in {elapsed:.3f} s: {elapsed / steps * 1e3:.1f} ms/step")
    log("kernel families (one untimed step, every kernel bracketed):")
    for name, e in sorted(breakdown.items(), key=lambda kv: -kv[1]["ms"]):
        tf = e["flops"] / (e["ms"] * 1e-3) / 1e12 if e["ms"] else 0.0
        gbs = e["bytes"] / (e["ms"] * 1e-3) / 1e9 if e["ms"] else 0.0
        log(f"  {name:28s} {e['launches']:5d}/step {e['ms']:9.2f} ms/step {tf:8.1f} TFLOP/s {gbs:8.1f} GB/s")
    d = timed[dominant]
    log(f"timed steps, {dominant}: {d['launches'] // steps}/step {d['ms'] / steps:.2f} ms/step "
        f"{d['flops'] / (d['ms'] * 1e-3) / 1e12:.1f} TFLOP/s")
    return elapsed / steps, breakdown, (dominant, d)


def measure_replay(dev, compiled, inputs, out, steps):
    """The same K steps replayed from one captured HIP graph
    (ndx_model_set_graph_replay), with no events at all: the first run
    records, the timed ones are one graph launch each."""
    compiled.SetGraphReplay(True)
    compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        compiled.DispatchInto(inputs, out)
    dev.Synchronize()
    elapsed = time.perf_counter() - t0
    compiled.SetGraphReplay(False)
    log(f"{steps} steps replayed from one HIP graph in {elapsed:.3f} s: {elapsed / steps * 1e3:.1f} ms/step")
    return elapsed / steps


def roofline(dominant, steps, peak, workload):
    """The dominant MFMA kernel family (GEMM, convolution or attention) by
    time: algorithmic flops per launch over its average launch, both from the
    events bracketing its launches in the timed steps."""
    name, dom = dominant
    per_launch = dom["flops"] / dom["launches"]
    avg_ms = dom["ms"] / dom["launches"]
    achieved = per_launch / (avg_ms * 1e-3) / 1e12
    traffic, src = read_traffic(name, workload)
    return {
        "bound": "mfma", "kernel": name, "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
        "frac": achieved / peak, "traffic": traffic, "traffic_unit": "bytes/launch", "traffic_source": src,
        "algorithmic_flop_per_launch": per_launch, "launches_per_step": dom["launches"] // steps,
        "avg_launch_ms": avg_ms,
    }


def setup_mmdit(args, dev, seed, DT):
    from naivediffusion_amd import mmdit, rng
    from naivediffusion_amd.tensors import HostTensor

    cfg = mmdit.MmditConfig(blocks=args.blocks or 60)
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    img_h, img_w = (int(v) for v in args.image.lower().split("x"))
    if img_h % 16 or img_w % 16:
        sys.exit("--image sides must be multiples of 16 (8x VAE, 2x2 patch)")
    B, lat_h, lat_w, nt = args.batch, img_h // 8, img_w // 8, 256
    gh, gw = lat_h // cfg.patch, lat_w // cfg.patch
    ni = gh * gw
    t0 = time.perf_counter()
    weights = mmdit.device_weights(dev, cfg, seed)
    log(f"synthetic weights on the device in {time.perf_counter() - t0:.1f} s")
    model = mmdit.build_step_model(dev, cfg, weights, B, nt, lat_h, lat_w, compute, args.int8,
                                   two_streams=not args.one_stream)
    n = ni + nt
    cos, sin = mmdit.rope_tables(gh, gw, nt)
    temb = np.tile(mmdit.time_embedding(0.5, cfg.time_dim), (B, 1)).reshape(B, 1, 1, cfg.time_dim)
    inputs = [
        dev.Normal(DT.Float32, [B, cfg.latent_channels, lat_h, lat_w], rng.tensor_seed(seed, "latent")),
        dev.Normal(DT.Float32, [B, 1, nt, cfg.text_dim], rng.tensor_seed(seed, "text")),
        dev.Upload(HostTensor.FromFloats(np.ascontiguousarray(temb, np.float32))),
        dev.Upload(HostTensor.FromFloats(cos.reshape(1, n, 1, 64))),
        dev.Upload(HostTensor.FromFloats(sin.reshape(1, n, 1, 64))),
    ]
    out = [dev.Empty(DT.Float32, [B, cfg.latent_channels, lat_h, lat_w])]
    wdesc = {None: f"{args.compute} weights", "block32": "int8 weights, fp16 scales per 32 columns",
             "channel": "int8 weights, fp32 scales per output channel"}[args.int8]
    return dict(
        model=model, inputs=inputs, out=out,
        metric="Qwen-Image DiT s/step @1024x1344 (bf16/int8 wts), 1 MI355X; % MFMA peak",
        config={"workload": (f"Qwen-Image-shaped MMDiT denoiser step, {cfg.blocks} dual-stream blocks, "
                             f"{img_h}x{img_w} (latent 16x{lat_h}x{lat_w}, 2x2 patch: {ni} image + {nt} text tokens), "
                             f"hidden 3072, 24x128 heads, MLP 12288, batch {B}, {args.compute} compute, {wdesc}"),
                "blocks": cfg.blocks, "image_tokens": ni, "text_tokens": nt, "batch": B,
                "weights": f"int8-{args.int8}" if args.int8 else args.compute,
                "streams": 1 if args.one_stream else 2},
        data="synthetic (seeded N(0,1) latent and text, N(0,0.02) bf16 weights made on the GPU)",
        cpu=lambda: cpu_baseline(dev, cfg, seed, ni, nt, (gh, gw), B),
    )


def setup_anima(args, dev, seed, DT):
    from naivediffusion_amd import anima, rng
    from naivediffusion_amd.layers import Transformer
    from naivediffusion_amd.tensors import HostTensor

    cfg = anima.AnimaConfig(blocks=args.blocks or 28)
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    store = compute if compute != DT.Float32 else DT.Float16
    lat, n_ctx = 128, 512
    n = (lat // 2) ** 2
    weights = anima.device_weights(dev, cfg, seed, store)
    model = anima.build_step_model(dev, cfg, weights, lat, lat, n_ctx, compute, bool(args.int8))
    cos, sin = anima.rope_tables(lat // 2, lat // 2, cfg.head_dim)
    half = cfg.head_dim // 2
    inputs = [
        dev.Normal(DT.Float32, [1, cfg.latent_channels, lat, lat], rng.tensor_seed(seed, "latent")),
        dev.Upload(HostTensor.FromFloats(Transformer.Sinusoid(0.5, cfg.width).reshape(1, 1, 1, cfg.width))),
        dev.Normal(DT.Float32, [1, 1, n_ctx, cfg.context_width], rng.tensor_seed(seed, "context")),
        dev.Upload(HostTensor.FromFloats(cos.reshape(1, n, 1, half))),
        dev.Upload(HostTensor.FromFloats(sin.reshape(1, n, 1, half))),
    ]
    out = [dev.Empty(DT.Float32, [1, cfg.latent_channels, lat, lat])]

    def cpu():
        import oracle
        names = list(anima.block_weight_shapes(cfg, 0))
        dw = anima.device_weights(dev, cfg, seed, DT.BFloat16, names)
        w = {k: t.Download().ToFloats() for k, t in dw.items()}
        for t in dw.values():
            t.Dispose()
        x = dev.Normal(DT.Float32, [n, cfg.width], rng.tensor_seed(seed, "cpu.x")).Download().ToFloats()
        ctx = inputs[2].Download().ToFloats().reshape(n_ctx, cfg.context_width)
        tmb = Transformer.Sinusoid(0.5, cfg.width)
        lora = np.zeros(3 * cfg.width, np.float32)
        threads = len(os.sched_getaffinity(0))
        t0 = time.perf_counter()
        oracle.anima_block(x, tmb, lora, ctx, w, 0, cfg.heads, cos, sin)
        dt = time.perf_counter() - t0
        return {"value": dt * cfg.blocks, "unit": "s/step", "cores": threads, "kind": "port",
                "sample": (f"one Anima block ({n} tokens, context {n_ctx}, hidden {cfg.width}, fp32) on the oracle "
                           f"in {dt:.2f} s, x{cfg.blocks} blocks (extrapolated)")}

    return dict(
        model=model, inputs=inputs, out=out,
        metric="Anima DiT s/step @1024x1024, 1 MI355X; % MFMA peak",
        config={"workload": (f"Anima-shaped 2B DiT denoiser step, {cfg.blocks} blocks, 1024x1024 (latent 16x{lat}x{lat}, "
                             f"2x2 patch: {n} tokens), hidden 2048, 16x128 heads, MLP 8192, cross-attention to "
                             f"{n_ctx}x1024 context, batch 1, {args.compute} compute"),
                "blocks": cfg.blocks, "tokens": n, "context_rows": n_ctx},
        data="synthetic (seeded N(0,1) latent and context, N(0,0.02) weights made on the GPU)",
        cpu=cpu,
    )


def setup_qwen(args, dev, seed, DT):
    from naivediffusion_amd import qwen, rng
    from naivediffusion_amd.tensors import HostTensor

    cfg = qwen.QwenImageConfig(blocks=args.blocks or 32)
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    store = compute if compute != DT.Float32 else DT.Float16
    lat, n_txt, real = 64, 256, 200
    n_img = lat * lat
    n = n_img + n_txt
    weights = qwen.device_weights(dev, cfg, seed, store)
    model = qwen.build_step_model(dev, cfg, weights, lat, lat, n_txt, compute, bool(args.int8))
    cond = qwen.conditioning(np.zeros((real, 1), np.float32), n_txt, lat, lat)
    times = np.stack([qwen.time_embedding(0.5, cfg.time_dim), qwen.time_embedding(0.0, cfg.time_dim)])
    inputs = [
        dev.Normal(DT.Float32, [1, cfg.latent_channels, lat, lat], rng.tensor_seed(seed, "latent")),
        dev.Upload(HostTensor.FromFloats(times.reshape(1, 1, 2, -1))),
        dev.Normal(DT.Float32, [1, 1, n_txt, cfg.context_width], rng.tensor_seed(seed, "context")),
        dev.Upload(HostTensor.FromInt32(cond["text_mask"], 1, 1, n_txt, n_txt)),
        dev.Upload(HostTensor.FromInt32(cond["key_length"], 1, 1, 1, 1)),
        dev.Upload(HostTensor.FromFloats(cond["cos"].reshape(1, n, 1, 64))),
        dev.Upload(HostTensor.FromFloats(cond["sin"].reshape(1, n, 1, 64))),
    ]
    out = [dev.Empty(DT.Float32, [1, cfg.latent_channels, lat, lat])]

    def cpu():
        import oracle
        names = list(qwen.block_weight_shapes(cfg, 0)) + [
            "time_text_embed.timestep_embedder.linear_1.weight", "time_text_embed.timestep_embedder.linear_2.weight",
            "modulation.1.weight"]
        dw = qwen.device_weights(dev, cfg, seed, DT.BFloat16, names)
        w = {k: t.Download().ToFloats().reshape(t.Shape) for k, t in dw.items()}
        for t in dw.values():
            t.Dispose()
        x = dev.Normal(DT.Float32, [n, cfg.width], rng.tensor_seed(seed, "cpu.x")).Download().ToFloats().reshape(n, -1)
        _, mod = oracle.qwen_modulation(0.5, w, cfg.time_dim, cfg.width)
        threads = len(os.sched_getaffinity(0))
        t0 = time.perf_counter()
        oracle.qwen_block(x, mod, w, 0, cfg.heads, n_img, cond["cos"], cond["sin"], int(cond["key_length"][0]),
                          cond["text_mask"])
        dt = time.perf_counter() - t0
        return {"value": dt * cfg.blocks, "unit": "s/step", "cores": threads, "kind": "port",
                "sample": (f"one Qwen-Image 2.1 block ({n_img} image + {n_txt} text tokens, width {cfg.width}, fp32) "
                           f"on the oracle in {dt:.2f} s, x{cfg.blocks} blocks (extrapolated)")}

    return dict(
        model=model, inputs=inputs, out=out,
        metric="Qwen-Image 2.1 DiT s/step @1024x1024, 1 MI355X; % MFMA peak",
        config={"workload": (f"Qwen-Image 2.1 single-stream DiT denoiser step, {cfg.blocks} blocks, 1024x1024 "
                             f"(latent 64x{lat}x{lat}, patch 1: {n_img} image + {n_txt} text rows, {real} real), "
                             f"hidden 4096, 32x128 heads, SwiGLU 12288, batch 1, {args.compute} compute"),
                "blocks": cfg.blocks, "image_tokens": n_img, "text_rows": n_txt},
        data="synthetic (seeded N(0,1) latent and context, N(0,0.02) weights made on the GPU)",
        cpu=cpu,
    )


def setup_sdxl(args, dev, seed, DT):
    from naivediffusion_amd import rng, sdxl
    from naivediffusion_amd.tensors import HostTensor

    cfg = sdxl.SdxlConfig()
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    B, lat, tokens = 2, 128, 77
    weights = sdxl.device_weights(dev, cfg, seed, compute)
    model = sdxl.build_unet(dev, cfg, weights, B, lat, lat, tokens, compute, bool(args.int8))
    t = np.tile(sdxl.timestep_embedding([500.0], cfg.block_out[0]), (B, 1)).reshape(B, 1, 1, -1)
    add = np.stack([sdxl.add_conditioning(np.zeros(cfg.pooled_width, np.float32), add_time_dim=cfg.add_time_dim)] * B)
    inputs = [
        dev.Normal(compute, [B, cfg.in_channels, lat, lat], rng.tensor_seed(seed, "latent")),
        dev.Upload(HostTensor.FromFloats(np.ascontiguousarray(t)).ConvertTo(compute)),
        dev.Upload(HostTensor.FromFloats(add.reshape(B, 1, 1, -1)).ConvertTo(compute)),
        dev.Normal(compute, [B, 1, tokens, cfg.context_width], rng.tensor_seed(seed, "context")),
    ]
    out = [dev.Empty(compute, [B, cfg.in_channels, lat, lat])]
    return dict(
        model=model, inputs=inputs, out=out,
        metric="SDXL UNet s/step @1024x1024 CFG batch 2, 1 MI355X; % MFMA peak",
        config={"workload": (f"SDXL UNet step, 1024x1024 (latent 4x{lat}x{lat}), CFG batch {B}, context {tokens}x2048, "
                             f"{args.compute} compute"), "batch": B},
        data="synthetic (seeded N(0,1) latent and context, N(0,0.02) weights made on the GPU)",
        cpu=None,
    )


def setup_vae(args, dev, seed, DT):
    from naivediffusion_amd import rng, vae

    cfg = vae.SDXL
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    side = 1024
    lat = side // cfg.scale_factor
    weights = vae.device_weights(dev, cfg, seed, compute)
    model = vae.build_decoder(dev, cfg, weights, side, side, compute)
    inputs = [dev.Normal(DT.Float32, [1, cfg.latent_channels, lat, lat], rng.tensor_seed(seed, "latent"), 0.0,
                         cfg.scaling_factor)]
    out = [dev.Empty(compute, [1, cfg.image_channels, side, side])]
    return dict(
        model=model, inputs=inputs, out=out,
        metric="SDXL VAE decode s/image @1024x1024, 1 MI355X; % MFMA peak",
        config={"workload": (f"SDXL VAE decoder (AutoencoderKL 128/256/512/512), latent 4x{lat}x{lat} -> "
                             f"3x{side}x{side}, {args.compute} compute"), "batch": 1},
        data="synthetic (seeded latent, N(0, 1/fan_in) weights made on the GPU)",
        cpu=None,
    )


def setup_wan22(args, dev, seed, DT):
    from naivediffusion_amd import rng, vae

    cfg = vae.WAN22
    compute = {"bf16": DT.BFloat16, "f32": DT.Float32, "f16": DT.Float16}[args.compute]
    side = 1024
    lat = side // cfg.scale_factor
    weights = vae.wan22_device_weights(dev, cfg, seed, compute)
    model = vae.build_wan22_decoder(dev, cfg, weights, side, side, compute)
    inputs = [dev.Normal(DT.Float32, [1, cfg.latent_channels, lat, lat], rng.tensor_seed(seed, "latent"))]
    out = [dev.Empty(compute, [1, 3, side, side])]
    return dict(
        model=model, inputs=inputs, out=out,
        metric="Qwen-Image 2.1 VAE (Wan 2.2) decode s/image @1024x1024, 1 MI355X; % MFMA peak",
        config={"workload": (f"Wan 2.2 VAE decoder on one frame (widths {'/'.join(map(str, cfg.widths))}), latent "
                             f"{cfg.latent_channels}x{lat}x{lat} -> 3x{side}x{side}, {args.compute} compute"),
                "batch": 1},
        data="synthetic (seeded N(0,1) latent, N(0, 1/fan_in) weights made on the GPU)",
        cpu=None,
    )


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=["mmdit", "anima", "sdxl", "qwen", "vae", "wan22"], default="mmdit",
                    help="mmdit (the headline), or the Anima DiT / SDXL UNet / Qwen-Image 2.1 steps, or the SDXL "
                         "(vae) / Qwen-Image 2.1 (wan22) VAE decodes")
    ap.add_argument("--compute", choices=["bf16", "f32", "f16"], default=None,
                    help="compute type (default bf16; fp16 for sdxl)")
    ap.add_argument("--int8", nargs="?", const="block32", default=None, choices=["block32", "channel"],
                    help="int8 weights: block32 (the reference's BlockQuantizer format, the default) or channel "
                         "(one fp32 scale per output channel)")
    ap.add_argument("--blocks", type=int, default=None, help="block count (default: the model's)")
    ap.add_argument("--image", default="1024x1344", help="mmdit: image size HxW (1328x1328 with --batch 2 and "
                    "--int8 channel is the CFG int8 configuration)")
    ap.add_argument("--batch", type=int, default=1, help="mmdit: batch (2: cond + uncond CFG)")
    ap.add_argument("--one-stream", action="store_true", help="mmdit: the text stream on the image stream's "
                    "stream (default: its own, beside the image stream)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-replay", action="store_true",
                    help="skip the steps replayed from one captured HIP graph (for profiler runs: rocprofv3's "
                         "kernel trace of the SDXL step's capture ended the process on the host)")
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
    if args.compute is None:
        args.compute = "f16" if args.workload == "sdxl" else "bf16"
    if args.workload != "mmdit" and (args.batch != 1 or args.image != "1024x1344"):
        sys.exit("--image and --batch apply to the mmdit workload only")

    import naivediffusion_amd as nd
    from naivediffusion_amd.tensors import HostDataType as DT

    seed = 20261201
    dev = nd.Device()
    log(f"device {dev.AdapterName}")
    t0 = time.perf_counter()
    setup = {"mmdit": setup_mmdit, "anima": setup_anima, "sdxl": setup_sdxl, "qwen": setup_qwen,
             "vae": setup_vae, "wan22": setup_wan22}[args.workload](
        args, dev, seed, DT)
    compiled = setup["model"].Compiled
    log(f"graph built and compiled in {time.perf_counter() - t0:.1f} s: {compiled.KernelCount} kernels/step, "
        f"{compiled.PersistentSize / 1e9:.1f} GB weights, {compiled.TemporarySize / 1e9:.2f} GB scratch")

    s_per_step, prof, dominant = measure(dev, compiled, setup["inputs"], setup["out"], args.steps, args.warmup)
    replay_s = None if args.no_replay else measure_replay(dev, compiled, setup["inputs"], setup["out"], args.steps)
    peak = FP32_PEAK_TFLOPS if args.compute == "f32" else MFMA_BF16_PEAK_TFLOPS
    total_flops = sum(e["flops"] for e in prof.values())
    kernel_ms = sum(e["ms"] for e in prof.values())

    cpu = None
    if not args.no_cpu_baseline and setup["cpu"] is not None:
        try:
            cpu = setup["cpu"]()
            log(f"cpu baseline {cpu['value']:.1f} s/step ({cpu['cores']} threads)")
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline failed: {e!r}")

    config = dict(setup["config"])
    config.update({
        "algorithmic_tflop_per_step": total_flops / 1e12,
        "achieved_tflops_step": total_flops / s_per_step / 1e12,
        "step_frac_of_mfma_peak": total_flops / s_per_step / 1e12 / peak,
        "kernel_ms_per_step": kernel_ms,
        # the same steps replayed from one captured HIP graph, no events (value: the event-bracketed run above)
        "graph_replay_ms_per_step": None if replay_s is None else replay_s * 1e3,
    })
    result = {
        "metric": setup["metric"],
        "value": s_per_step,
        "unit": "s/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": s_per_step * 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.compute,
        "data": setup["data"],
        "config": config,
        "roofline": roofline(dominant, args.steps, peak, args.workload),
        # From one untimed step with every kernel bracketed (two events per
        # kernel and a wait: the breakdown, not the timed step).
        "kernels": {k: {"ms_per_step": v["ms"], "launches_per_step": v["launches"],
                        "tflops": (v["flops"] / (v["ms"] * 1e-3) / 1e12) if v["ms"] else 0.0,
                        "gbs": (v["bytes"] / (v["ms"] * 1e-3) / 1e9) if v["ms"] else 0.0}
                    for k, v in prof.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
