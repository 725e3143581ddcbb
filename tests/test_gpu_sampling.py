"""The sampler on the device (ndx_op_guided_euler_step and sampling.sample):
the fused guidance combine + Euler step bit-exact with the oracle's float32
restatement of GuidanceStrategy.Combine and EulerScheduler.Step, with and
without the unconditional branch, on ragged sizes; and a three-step flow
Euler run with classifier-free guidance over a small MMDiT whose latent never
leaves the GPU, equal bit for bit to the reference's loop (Predict per branch
on host tensors, combine and step on the host) and within 1e-3 of the same
loop run entirely on the oracle (fp32 compute)."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import mmdit, rng, sampling
from naivediffusion_amd.graph import Ops
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(1, 16, 128, 168), (1, 3, 5, 7), (1, 64, 64, 64)])
@pytest.mark.parametrize("branches", [1, 2])
def test_guided_euler_step_is_bit_exact(device, shape, branches):
    print(f"[gpu] guided euler step {shape} branches={branches}", flush=True)
    g = np.random.default_rng(sum(shape) + branches)
    x, u, c = (g.standard_normal(shape).astype(np.float32) for _ in range(3))
    guidance, sigma, sigma_next = 3.5, 0.80125, 0.6515
    graph = nd.Graph(device)
    xi = graph.Input(DT.Float32, list(shape))
    ui = graph.Input(DT.Float32, list(shape)) if branches == 2 else None
    ci = graph.Input(DT.Float32, list(shape))
    si = graph.Input(DT.Float32, [1, 1, 1, 4])
    model = nd.CompiledModel(graph, [Ops.GuidedEulerStep(xi, ui, ci, si)], device)
    ins = [HostTensor.FromFloats(x)] + ([HostTensor.FromFloats(u)] if branches == 2 else []) + [
        HostTensor.FromFloats(c), HostTensor.FromFloats(np.array([guidance, sigma, sigma_next, 0], np.float32), 1, 1, 1, 4)]
    got = model.Dispatch(ins)[0].ToFloats().reshape(shape)
    model.Dispose()
    p = oracle.cfg_combine(u, c, guidance) if branches == 2 else c
    exp = oracle.euler_step(x, p, sigma, sigma_next)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


TINY = mmdit.MmditConfig(width=256, heads=2, mlp=512, blocks=2, latent_channels=16, patch=2, text_dim=64,
                         time_dim=32)


def test_device_sampling_loop(device):
    cfg, H, W, nt, guidance, steps = TINY, 12, 16, 8, 4.0, 3
    w = mmdit.synthetic_weights(cfg, 81, norm_spread=0.1)
    latent = rng.normal(rng.tensor_seed(81, "noise"), (1, cfg.latent_channels, H, W))
    texts = [rng.normal(rng.tensor_seed(81, f"text{b}"), (1, 1, nt, cfg.text_dim)) for b in range(2)]
    _, sigmas = sampling.set_timesteps(sampling.FlowShiftSchedule(3.0), steps, "linspace")
    den = mmdit.QwenImageMmdit(device, cfg, w, H, W, nt, DT.Float32)
    compiled = den.model.Compiled
    n = den.cos.shape[0]
    print("[gpu] sampling loop on the device", flush=True)
    text_dev = [device.Upload(HostTensor.FromFloats(t)) for t in texts]
    cos = device.Upload(HostTensor.FromFloats(den.cos.reshape(1, n, 1, 64)))
    sin = device.Upload(HostTensor.FromFloats(den.sin.reshape(1, n, 1, 64)))
    tsin = [device.Upload(HostTensor.FromFloats(mmdit.time_embedding(float(s), cfg.time_dim).reshape(1, 1, 1, -1)))
            for s in sigmas[:-1]]
    preds = [device.Empty(DT.Float32, [1, cfg.latent_channels, H, W]) for _ in range(2)]

    def predict(x, step):
        for b in range(2):
            compiled.DispatchInto([x, text_dev[b], tsin[step], cos, sin], [preds[b]])
        return preds

    x0 = device.Upload(HostTensor.FromFloats(latent))
    final = sampling.sample(device, predict, x0, sigmas, guidance, 2).Download().ToFloats().reshape(latent.shape)
    print("[gpu] the reference's loop: Predict per branch, combine and step on the host", flush=True)
    x = latent.copy()
    for step in range(steps):
        u, c = (den.Predict(HostTensor.FromFloats(x), 0, float(sigmas[step]), {"context": t}).ToFloats()
                .reshape(x.shape) for t in texts)
        x = oracle.euler_step(x, oracle.cfg_combine(u, c, guidance), sigmas[step], sigmas[step + 1])
    assert np.array_equal(final.view(np.uint32), x.view(np.uint32))
    print("[gpu] the loop on the oracle", flush=True)
    y = latent.copy()
    for step in range(steps):
        u, c = (oracle.mmdit_step(y, t, float(sigmas[step]), w, cfg.blocks, cfg.heads, den.cos, den.sin, cfg.patch,
                                  cfg.eps) for t in texts)
        y = oracle.euler_step(y, oracle.cfg_combine(u, c, guidance), sigmas[step], sigmas[step + 1])
    err = rel_err(final, y)
    print(f"[gpu]   final latent vs the oracle loop {err:.2e}", flush=True)
    assert err <= 1e-3
    assert rel_err(final, latent) > 1e-2
    den.model.Dispose()
