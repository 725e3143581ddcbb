"""Graph replay (ndx_model_set_graph_replay) against eager runs: the whole
run, both streams, recorded once as a HIP graph and replayed must give the
eager run's outputs bit for bit, on every replay, with eager work and
synchronisations of the program between replays; new values in the same
input tensors are seen by the replay; other output tensors record the graph
again. Covers a two-stream MMDiT block (joint attention, key-split partials
in the arena) and a small SDXL UNet (split GroupNorm statistics, the
convolutions' layout copies)."""

import numpy as np
import pytest

import naivediffusion_amd as nd
from naivediffusion_amd import mmdit, rng, sdxl
from naivediffusion_amd.graph import Ops
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor

pytestmark = pytest.mark.gpu

CFG = mmdit.MmditConfig(width=1024, heads=8, mlp=2048, blocks=1)


def mmdit_case(device):
    w = mmdit.synthetic_weights(CFG, 3, list(mmdit.block_weight_shapes(CFG, 0)), norm_spread=0.1)
    ni, nt, D = 512, 64, CFG.width
    compiled = mmdit.build_block_model(device, CFG, w, 1, ni, nt, DT.BFloat16).Compiled
    cos, sin = mmdit.rope_tables(16, 32, nt)
    n = ni + nt

    def inputs(seed):
        host = [rng.normal(rng.tensor_seed(seed, "xi"), (1, 1, ni, D)), rng.normal(rng.tensor_seed(seed, "xt"), (1, 1, nt, D)),
                rng.normal(rng.tensor_seed(seed, "t"), (1, 1, 1, D)), cos.reshape(1, n, 1, 64), sin.reshape(1, n, 1, 64)]
        return [HostTensor.FromFloats(a) for a in host]

    return compiled, inputs, [(DT.Float32, [1, 1, ni, D]), (DT.Float32, [1, 1, nt, D])]


def unet_case(device):
    cfg = sdxl.SdxlConfig(block_out=(64, 128, 128), transformer_layers=(0, 1, 1), heads=(1, 2, 2), context_width=64,
                          time_embed=256, add_time_dim=32, pooled_width=128)
    w = sdxl.synthetic_weights(cfg, 4, DT.Float16)
    B, H, W, tokens = 2, 16, 16, 8
    compiled = sdxl.build_unet(device, cfg, w, B, H, W, tokens, DT.Float16).Compiled

    def inputs(seed):
        host = [rng.normal(rng.tensor_seed(seed, "s"), (B, cfg.in_channels, H, W)),
                np.tile(sdxl.timestep_embedding([500.0], cfg.block_out[0]), (B, 1)).reshape(B, 1, 1, -1),
                rng.normal(rng.tensor_seed(seed, "a"), (B, 1, 1, cfg.add_width)),
                rng.normal(rng.tensor_seed(seed, "c"), (B, 1, tokens, cfg.context_width))]
        return [HostTensor.FromFloats(np.ascontiguousarray(a, np.float32)).ConvertTo(DT.Float16) for a in host]

    return compiled, inputs, [(DT.Float16, [B, cfg.in_channels, H, W])]


def read(device, outs):
    device.Synchronize()
    return [o.Download().Data.copy() for o in outs]


def copier(device, tensors):
    """Writes new values into existing device tensors: an identity model per
    tensor whose output is bound to it."""
    models = []
    for t in tensors:
        g = nd.Graph(device)
        x = g.Input(t.DataType, list(t.Shape))
        models.append(nd.CompiledModel(g, [Ops.Identity(x)], device))

    def put(dst, srcs):
        for m, d, s in zip(models, dst, srcs):
            m.DispatchInto([s], [d])
    return put


@pytest.mark.parametrize("case", [mmdit_case, unet_case], ids=["mmdit-two-streams", "sdxl-unet"])
def test_replay_equals_eager(device, case):
    compiled, inputs, out_specs = case(device)
    print(f"[gpu] graph replay: {case.__name__}", flush=True)
    src = {k: [device.Upload(t) for t in inputs(k)] for k in (1, 2)}
    outs = [device.Empty(dt, s) for dt, s in out_specs]
    eager = {}
    for k in (1, 2):
        compiled.DispatchInto(src[k], outs)
        eager[k] = read(device, outs)
    assert not np.array_equal(eager[1][0], eager[2][0])
    ins = [device.Upload(t) for t in inputs(1)]
    put = copier(device, ins)
    # Eager work of the program's own between replays: a small model.
    g = nd.Graph(device)
    x = g.Input(DT.Float32, [1, 1, 64, 64])
    side = nd.CompiledModel(g, [x * 2.0], device)
    side_in = device.Upload(HostTensor.FromFloats(np.ones((1, 1, 64, 64), np.float32)))
    compiled.SetGraphReplay(True)
    for rep in range(6):
        k = 1 + rep % 2  # the same input tensors, other values each time
        put(ins, src[k])
        compiled.DispatchInto(ins, outs)
        for a, b in zip(read(device, outs), eager[k]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"replay {rep}"
        side.DispatchOnDevice([side_in])[0].Dispose()
        device.Synchronize()
    # Other output tensors: recorded again, still the eager result.
    outs2 = [device.Empty(dt, s) for dt, s in out_specs]
    for _ in range(2):
        compiled.DispatchInto(ins, outs2)
        for a, b in zip(read(device, outs2), eager[2]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    compiled.SetGraphReplay(False)
    compiled.DispatchInto(src[1], outs)
    for a, b in zip(read(device, outs), eager[1]):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
