"""The allocation-free run (ndx_model_run_into_static_async) against the
ordinary one (ndx_model_run_into_async) through the C ABI: the same kernels
with the temporaries in the library's static scratch instead of the model's
arena give the same outputs bit for bit, on consecutive calls whose second
model is smaller (the array keeps the first call's contents), for a model
with attention and one with a split GroupNorm and convolutions; a model
whose temporaries exceed the array is refused."""

import numpy as np
import pytest

import naivediffusion_amd as nd
from naivediffusion_amd import mmdit, rng, sdxl
from naivediffusion_amd.layers import Layers
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from naivediffusion_amd.weights import WeightSet

pytestmark = pytest.mark.gpu

CFG = mmdit.MmditConfig(width=1024, heads=8, mlp=2048, blocks=1)


def mmdit_case(device, ni, nt, grid, seed):
    w = mmdit.synthetic_weights(CFG, seed, list(mmdit.block_weight_shapes(CFG, 0)), norm_spread=0.1)
    model = mmdit.build_block_model(device, CFG, w, 1, ni, nt, DT.BFloat16)
    D, n = CFG.width, ni + nt
    cos, sin = mmdit.rope_tables(grid[0], grid[1], nt)
    host = [rng.normal(rng.tensor_seed(seed, "xi"), (1, 1, ni, D)), rng.normal(rng.tensor_seed(seed, "xt"), (1, 1, nt, D)),
            rng.normal(rng.tensor_seed(seed, "t"), (1, 1, 1, D)), cos.reshape(1, n, 1, 64), sin.reshape(1, n, 1, 64)]
    ins = [device.Upload(HostTensor.FromFloats(a)) for a in host]
    return model.Compiled, ins, [[1, 1, ni, D], [1, 1, nt, D]]


def resnet_case(device, size, seed):
    cfg = sdxl.SdxlConfig()
    prefix = "down_blocks.1.resnets.0"
    w = {k: np.asarray(sdxl._init(k, s, seed), np.float32) for k, s in sdxl.weight_shapes(cfg).items()
         if k.startswith(prefix + ".")}
    model = nd.ModelBuilder(device, DT.Float16)
    W = WeightSet(model, w, DT.Float16, device)
    x = model.Placeholder([2, 320, size, size], DT.Float16)
    t = model.Placeholder([2, 1, 1, cfg.time_embed], DT.Float16)
    model.Compile([sdxl.resnet_block(model, W, cfg, x, Layers.Silu(t), prefix)])
    ins = [device.Upload(HostTensor.FromFloats(rng.normal(rng.tensor_seed(seed, "x"), (2, 320, size, size)))
                         .ConvertTo(DT.Float16)),
           device.Upload(HostTensor.FromFloats(rng.normal(rng.tensor_seed(seed, "t"), (2, 1, 1, cfg.time_embed)))
                         .ConvertTo(DT.Float16))]
    return model.Compiled, ins, [[2, 640, size, size]]


def outputs_of(device, compiled, ins, shapes, static):
    dtype = DT.Float32 if len(shapes) == 2 else DT.Float16
    outs = [device.Empty(dtype, s) for s in shapes]
    if static:
        compiled.DispatchIntoStatic(ins, outs)
    else:
        compiled.DispatchInto(ins, outs)
    device.Synchronize()
    return [o.Download().Data.copy() for o in outs]


@pytest.mark.parametrize("kind", ["mmdit", "resnet"])
def test_static_run_equals_the_arena_run(device, kind):
    if kind == "mmdit":
        big = mmdit_case(device, 512, 64, (16, 32), 1)
        small = mmdit_case(device, 128, 32, (8, 16), 2)
    else:
        big = resnet_case(device, 48, 3)
        small = resnet_case(device, 20, 4)
    for name, (compiled, ins, shapes) in (("big", big), ("small", small)):
        print(f"[gpu] static run: {kind} {name}, temporary {compiled.TemporarySize} bytes", flush=True)
        assert 0 < compiled.TemporarySize <= compiled.STATIC_SCRATCH_BYTES
    ref = [outputs_of(device, c, i, s, False) for c, i, s in (big, small)]
    # Two calls in a row, the second with the smaller model; then the first
    # again over what the second left in the array.
    for case, want in ((big, ref[0]), (small, ref[1]), (big, ref[0])):
        got = outputs_of(device, *case, True)
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_static_run_refuses_a_model_beyond_the_array(device):
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, 1, 4096, 8192])
    m = nd.CompiledModel(g, [(x * 2.0) * 3.0], device)
    assert m.TemporarySize > m.STATIC_SCRATCH_BYTES
    with pytest.raises(nd.ArgumentError, match="static scratch"):
        m.DispatchIntoStatic([device.Empty(DT.Float32, [1, 1, 4096, 8192])],
                             [device.Empty(DT.Float32, [1, 1, 4096, 8192])])
