"""GPU parity of Qwen-Image 2.1's single-stream denoiser (Models/QwenImage/
QwenImageDit.cs) against the oracle's composition, which a float64 block
with the reference's own pair rotation pins: one block at the model's width
(4096, 32 heads of 128, SwiGLU 12288) with 1024 image tokens and 64 text rows
of which 50 are real (the image rows read every real key, the text rows the
causal table; the padding never reaches a real row), at bf16 (2e-2) and fp32
(1e-3) compute, with weights made on the device (so PairsToHalves and the
gate/up interleave run there); and a small whole step (embeddings, time path,
two blocks, final layer) with host weights. Tolerance: max|gpu - oracle| /
max|oracle| of the block's update (or the step's flow)."""

import numpy as np
import pytest

import oracle
from naivediffusion_amd import qwen, rng
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu

FULL = qwen.QwenImageConfig(blocks=1)
TIME = ["time_text_embed.timestep_embedder.linear_1.weight", "time_text_embed.timestep_embedder.linear_2.weight",
        "modulation.1.weight"]


def say(msg):
    print(f"[gpu] {msg}", flush=True)


def normal(device, seed, name, shape, std=1.0):
    t = device.Normal(DT.Float32, shape, rng.tensor_seed(seed, name), 0.0, std)
    a = t.Download().ToFloats().reshape(shape)
    t.Dispose()
    return a


def block_names():
    return list(qwen.block_weight_shapes(FULL, 0)) + TIME


@pytest.fixture(scope="module")
def full_block(device):
    cfg = FULL
    lat, n_txt, real = 32, 64, 50
    n_img = lat * lat
    N = n_img + n_txt
    say("qwen block: weights on the device, oracle copy downloaded")
    dw = qwen.device_weights(device, cfg, 71, DT.BFloat16, block_names())
    w = {k: t.Download().ToFloats().reshape(t.Shape) for k, t in dw.items()}
    for t in dw.values():
        t.Dispose()
    # the head norms off 1, so their permutation matters
    for k in ("transformer_blocks.0.attn.norm_q.weight", "transformer_blocks.0.attn.norm_k.weight"):
        w[k] = (1 + rng.normal(rng.tensor_seed(71, k), (128,), 0.0, 0.1)).astype(np.float32)
        w[k] = HostTensor.FromFloats(w[k]).ConvertTo(DT.BFloat16).ToFloats()
    x = normal(device, 71, "x", (N, cfg.width))
    cond = qwen.conditioning(np.zeros((real, 8), np.float32), n_txt, lat, lat)
    sigma = 0.6
    time = np.stack([qwen.time_embedding(sigma, cfg.time_dim), qwen.time_embedding(0.0, cfg.time_dim)])
    _, mod = oracle.qwen_modulation(sigma, w, cfg.time_dim, cfg.width)
    say("qwen block: oracle (1024 + 64 tokens, width 4096)")
    ref = oracle.qwen_block(x, mod, w, 0, cfg.heads, n_img, cond["cos"], cond["sin"], int(cond["key_length"][0]),
                            cond["text_mask"])
    return w, x, time, cond, ref, n_img, n_txt


def device_copy(device, w):
    """The weights as device bf16 tensors (the builder takes them over)."""
    return {k: device.Upload(HostTensor.FromFloats(v).ConvertTo(DT.BFloat16)) for k, v in w.items()}


@pytest.mark.parametrize("compute,tol,fuse", [(DT.BFloat16, 2e-2, "0"), (DT.Float32, 1e-3, "0"),
                                              (DT.BFloat16, 2e-2, "1")])
def test_qwen_block_at_model_width(device, full_block, compute, tol, fuse, monkeypatch):
    """The block against the oracle; with NDX_FUSE_QK_NORM=1 the head norms
    run in the QKV projection's epilogue and the attention reads query
    chunks of the projection's rows (views re-expressed over its buffer)."""
    monkeypatch.setenv("NDX_FUSE_QK_NORM", fuse)
    w, x, time, cond, ref, n_img, n_txt = full_block
    N = n_img + n_txt
    say(f"qwen block {compute.name} fused head norm {fuse}")
    model = qwen.build_block_model(device, FULL, device_copy(device, w), n_img, n_txt, compute)
    out = model.Run(HostTensor.FromFloats(x.reshape(1, 1, N, -1)), HostTensor.FromFloats(time.reshape(1, 1, 2, -1)),
                    HostTensor.FromInt32(cond["text_mask"], 1, 1, n_txt, n_txt),
                    HostTensor.FromInt32(cond["key_length"], 1, 1, 1, 1),
                    HostTensor.FromFloats(cond["cos"].reshape(1, N, 1, 64)),
                    HostTensor.FromFloats(cond["sin"].reshape(1, N, 1, 64)))[0].ToFloats().reshape(N, -1)
    model.Dispose()
    real = int(cond["key_length"][0])
    err = rel_err(out[:real] - x[:real], ref[:real] - x[:real])
    err_all = rel_err(out - x, ref - x)
    say(f"  update rel err {err:.2e} over the real rows, {err_all:.2e} over all (bound {tol})")
    assert err <= tol and err_all <= tol


SMALL = qwen.QwenImageConfig(width=256, heads=2, mlp=384, blocks=2, latent_channels=64, context_width=128, time_dim=64)


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_qwen_step_small(device, compute, tol):
    cfg = SMALL
    H, W, n_txt, real = 8, 10, 16, 12
    say(f"qwen step (width 256, 2 blocks) {compute.name}")
    w = qwen.synthetic_weights(cfg, 72, norm_spread=0.1)
    latent = rng.normal(rng.tensor_seed(72, "latent"), (cfg.latent_channels, H, W))
    ctx = rng.normal(rng.tensor_seed(72, "ctx"), (real, cfg.context_width))
    cond = qwen.conditioning(ctx, n_txt, H, W)
    den = qwen.QwenImageDit(device, cfg, w, H * 16, W * 16, n_txt, compute)
    flow = den.Predict(HostTensor.FromFloats(latent), 500, 0.45, cond).ToFloats().reshape(latent.shape)
    den.Dispose()
    ref = oracle.qwen_step(latent, 0.45, cond["context"], cond["text_mask"], int(cond["key_length"][0]), w,
                           cfg.blocks, cfg.heads, cond["cos"], cond["sin"], cfg.time_dim)
    err = rel_err(flow, ref)
    say(f"  rel err {err:.2e} (bound {tol})")
    assert err <= tol
