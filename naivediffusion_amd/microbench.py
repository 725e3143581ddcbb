"""Standalone timing of the bandwidth-bound kernels at the 60-block MMDiT
step's shapes (5376 image + 256 text tokens, hidden 3072), each in a graph of
its own, so their rates can be read apart from the step's two streams:

- modulate: Transformer.Modulate (LayerNorm, then (1 + scale) and shift,
  rounded to bf16) of the fp32 residual stream, image and text rows;
- adaln_gemv: the per-block adaLN projection, SiLU(temb) [1, 3072] times
  [18432, 3072] bf16 plus an fp32 bias (M = 1: a weight-streaming GEMV);
- head_norm_rotate: the per-head RMSNorm + fp32 RoPE of Q read out of the
  packed QKV projection;
- gemm_qkv / gemm_out / gemm_fc1 / gemm_fc2: the image stream's four
  projections alone (rates in TFLOP/s).

Every launch is bracketed by HIP events on the stream it runs on; the
printed rate is the algorithmic bytes per launch over the mean launch time.

    python -m naivediffusion_amd.microbench [--ops modulate,adaln_gemv,...] [--reps N]
"""

from __future__ import annotations

import argparse
import json

import numpy as np

from . import rng
from .graph import CompiledModel, Graph, Ops
from .layers import Layers, Transformer
from .mmdit import rope_tables
from .tensors import Device, HostDataType as DT, HostTensor

D, H, NI, NT = 3072, 24, 5376, 256


def _modulate(dev, rows):
    g = Graph(dev, DT.BFloat16)
    x = g.Input(DT.Float32, [1, 1, rows, D])
    mod = g.Input(DT.Float32, [1, 1, 1, 6 * D])
    shift = Ops.Slice(mod, [0, 0, 0, 0], [1, 1, 1, D])
    scale = Ops.Slice(mod, [0, 0, 0, D], [1, 1, 1, D])
    out = Ops.Modulate(x, shift, scale, 1e-6, DT.BFloat16)
    ins = [dev.Normal(DT.Float32, [1, 1, rows, D], 1), dev.Normal(DT.Float32, [1, 1, 1, 6 * D], 2, 0.0, 0.1)]
    return CompiledModel(g, [out], dev), ins, rows * D * 4 + 2 * D * 4 + rows * D * 2


def _adaln_gemv(dev, rows=1):
    from .graph import ModelBuilder
    m = ModelBuilder(dev, DT.BFloat16)
    t = m.Placeholder([1, 1, rows, D], DT.Float32)
    w = m.WeightOnDevice(dev.Normal(DT.BFloat16, [6 * D, D], 3, 0.0, 0.02), 6 * D)
    b = m.ConstantOnDevice(dev.Normal(DT.Float32, [6 * D], 4, 0.0, 0.02))
    y = Layers.Linear(m, Layers.Silu(t), w, b)
    m.Compile([y])
    return m.Compiled, [dev.Normal(DT.Float32, [1, 1, rows, D], 5)], 6 * D * D * 2


def _head_norm_rotate(dev, rows):
    g = Graph(dev, DT.BFloat16)
    qkv = g.Input(DT.BFloat16, [1, 1, rows, 3 * D])
    w = g.Input(DT.BFloat16, [128])
    cos = g.Input(DT.Float32, [1, rows, 1, 64])
    sin = g.Input(DT.Float32, [1, rows, 1, 64])
    q = Ops.Slice(qkv, [0, 0, 0, 0], [1, 1, rows, D])
    out = Ops.HeadNormRotate(q, w, 1e-6, cos, sin, H, DT.BFloat16)
    c, s = rope_tables(64, rows // 64, 0)
    ins = [dev.Normal(DT.BFloat16, [1, 1, rows, 3 * D], 6),
           dev.Upload(HostTensor.FromFloats(np.ones(128, np.float32)).ConvertTo(DT.BFloat16)),
           dev.Upload(HostTensor.FromFloats(c.reshape(1, rows, 1, 64))),
           dev.Upload(HostTensor.FromFloats(s.reshape(1, rows, 1, 64)))]
    return CompiledModel(g, [out], dev), ins, rows * D * 2 * 2 + rows * 64 * 4 * 2


def _gemm(dev, M, N, K):
    """One image-stream projection: x [M, K] bf16 times W [N, K] bf16."""
    from .graph import ModelBuilder
    m = ModelBuilder(dev, DT.BFloat16)
    x = m.Placeholder([1, 1, M, K], DT.BFloat16)
    w = m.WeightOnDevice(dev.Normal(DT.BFloat16, [N, K], 7, 0.0, 0.02), N)
    m.Compile([Layers.Linear(m, x, w)])
    return m.Compiled, [dev.Normal(DT.BFloat16, [1, 1, M, K], 8)], 2.0 * M * N * K


CASES = {
    "modulate_img": lambda dev: _modulate(dev, NI),
    "modulate_txt": lambda dev: _modulate(dev, NT),
    "adaln_gemv": _adaln_gemv,
    "head_norm_rotate_img": lambda dev: _head_norm_rotate(dev, NI),
    # the image stream's four products (flops, not bytes, per launch)
    "gemm_qkv": lambda dev: _gemm(dev, NI, 3 * D, D),
    "gemm_out": lambda dev: _gemm(dev, NI, D, D),
    "gemm_fc1": lambda dev: _gemm(dev, NI, 4 * D, D),
    "gemm_fc2": lambda dev: _gemm(dev, NI, D, 4 * D),
}
FLOP_CASES = {"gemm_qkv", "gemm_out", "gemm_fc1", "gemm_fc2"}


def run(ops, reps: int = 50, warmup: int = 5):
    results = {}
    with Device() as dev:
        for name in ops:
            compiled, ins, nbytes = CASES[name](dev)
            outs = compiled.DispatchOnDevice(ins)
            for _ in range(warmup):
                compiled.DispatchInto(ins, outs)
            dev.Synchronize()
            compiled.SetProfiling(True)
            for _ in range(reps):
                compiled.DispatchInto(ins, outs)
            prof = compiled.Profile()
            compiled.SetProfiling(False)
            fam, e = max(prof.items(), key=lambda kv: kv[1]["ms"])
            us = e["ms"] / e["launches"] * 1e3
            if name in FLOP_CASES:
                results[name] = {"kernel": fam, "us_per_launch": us, "flop_per_launch": nbytes,
                                 "TFLOP_per_s": nbytes / (us * 1e-6) / 1e12, "launches": e["launches"]}
                print(f"{name:22s} {fam:34s} {us:9.2f} us {nbytes / 1e9:9.2f} GF "
                      f"{nbytes / (us * 1e-6) / 1e12:8.1f} TFLOP/s", flush=True)
            else:
                results[name] = {"kernel": fam, "us_per_launch": us, "bytes_per_launch": nbytes,
                                 "GB_per_s": nbytes / (us * 1e-6) / 1e9, "launches": e["launches"]}
                print(f"{name:22s} {fam:34s} {us:9.2f} us {nbytes / 1e6:9.2f} MB "
                      f"{nbytes / (us * 1e-6) / 1e9:8.1f} GB/s", flush=True)
            for t in outs:
                t.Dispose()
            compiled.Dispose()
    return results


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--ops", default=",".join(CASES), help="comma-separated: " + ", ".join(CASES))
    ap.add_argument("--reps", type=int, default=50)
    ap.add_argument("--json", action="store_true", help="print one JSON line of the results at the end")
    args = ap.parse_args()
    res = run([o for o in args.ops.split(",") if o], args.reps)
    if args.json:
        print(json.dumps(res))


if __name__ == "__main__":
    main()
