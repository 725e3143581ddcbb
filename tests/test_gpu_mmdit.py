"""GPU parity of the Qwen-Image-shaped MMDiT: the dual-stream joint block at
its real shape (hidden 3072, 24 x 128 heads, MLP 12288, 1024 image + 128
text tokens, the first configuration of the benchmark) against the
oracle's composition of the reference primitives, at bf16 compute (2e-2),
fp32 compute (1e-3) and with int8 block-quantised weights; the CFG batch of
two against two batch-1 oracle runs; a padded text stream under the
key-length mask; and a small full denoiser step (embeddings, blocks, final
layer) against the oracle."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import mmdit, rng
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu

C0 = mmdit.MmditConfig(blocks=1)


def stream_weights(w, i, s):
    p = f"blocks.{i}.{s}"
    return dict(w_mod=w[f"{p}_mod.weight"], b_mod=w[f"{p}_mod.bias"], w_qkv=w[f"{p}_qkv.weight"],
                b_qkv=w[f"{p}_qkv.bias"], norm_q=w[f"{p}_norm_q.weight"], norm_k=w[f"{p}_norm_k.weight"],
                w_o=w[f"{p}_out.weight"], b_o=w[f"{p}_out.bias"], w_fc1=w[f"{p}_fc1.weight"],
                b_fc1=w[f"{p}_fc1.bias"], w_fc2=w[f"{p}_fc2.weight"], b_fc2=w[f"{p}_fc2.bias"])


def dequantized(w):
    """The weights as the int8 path sees them: quantised per 32 columns with
    fp16 scales, then multiplied back (ModelBuilder.Weight's format)."""
    out = {}
    for k, v in w.items():
        if v.ndim == 2 and v.size >= (1 << 16) and v.shape[1] % 32 == 0:
            q, s = oracle.quantize(v, v.shape[0])
            out[k] = (q.astype(np.float32).reshape(v.shape[0], -1, 32) *
                      oracle.f16_bits_to_f32(s)[:, :, None]).reshape(v.shape)
        else:
            out[k] = v
    return out


def block_case(cfg, ni, nt, grid, batch=1, seed=11):
    names = list(mmdit.block_weight_shapes(cfg, 0))
    w = mmdit.synthetic_weights(cfg, seed, names, norm_spread=0.1)
    D = cfg.width
    xi = rng.normal(rng.tensor_seed(seed, "x_img"), (batch, 1, ni, D))
    xt = rng.normal(rng.tensor_seed(seed, "x_txt"), (batch, 1, nt, D))
    temb = rng.normal(rng.tensor_seed(seed, "temb"), (batch, 1, 1, D))
    cos, sin = mmdit.rope_tables(grid[0], grid[1], nt)
    return w, xi, xt, temb, cos, sin


def run_block(device, cfg, w, xi, xt, temb, cos, sin, compute, int8=False, key_len=None, two_streams=True):
    B, _, ni, D = xi.shape
    nt = xt.shape[2]
    n = ni + nt
    model = mmdit.build_block_model(device, cfg, w, B, ni, nt, compute, int8, key_len=key_len is not None,
                                    two_streams=two_streams)
    ins = [HostTensor.FromFloats(xi), HostTensor.FromFloats(xt), HostTensor.FromFloats(temb),
           HostTensor.FromFloats(cos.reshape(1, n, 1, 64)), HostTensor.FromFloats(sin.reshape(1, n, 1, 64))]
    if key_len is not None:
        ins.append(HostTensor.FromInt32(np.array([key_len]), 1, 1, 1, 1))
    yi, yt = model.Run(*ins)
    model.Dispose()
    return yi.ToFloats(), yt.ToFloats()


def oracle_block(cfg, w, xi, xt, temb, cos, sin, key_len=-1):
    yi, yt = oracle.mmdit_block(xi.reshape(-1, cfg.width), xt.reshape(-1, cfg.width), temb.ravel(),
                                stream_weights(w, 0, "img"), stream_weights(w, 0, "txt"), cfg.heads, cos, sin,
                                key_len, cfg.eps)
    return yi, yt


@pytest.fixture(scope="module")
def config0():
    w, xi, xt, temb, cos, sin = block_case(C0, 1024, 128, (32, 32))
    print("[gpu] oracle: config-0 block (1024 + 128 tokens)", flush=True)
    ref = oracle_block(C0, w, xi, xt, temb, cos, sin)
    return w, xi, xt, temb, cos, sin, ref


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_config0_block(device, config0, compute, tol):
    w, xi, xt, temb, cos, sin, (ri, rt) = config0
    print(f"[gpu] config-0 block {compute.name}", flush=True)
    yi, yt = run_block(device, C0, w, xi, xt, temb, cos, sin, compute)
    ei, et = rel_err(yi.reshape(ri.shape), ri), rel_err(yt.reshape(rt.shape), rt)
    print(f"[gpu]   image {ei:.2e} text {et:.2e}", flush=True)
    assert ei <= tol and et <= tol
    # the block must have changed the streams, not passed them through
    assert rel_err(xi.reshape(ri.shape), ri) > 10 * tol


def test_config0_block_int8(device, config0):
    w, xi, xt, temb, cos, sin, (ri, rt) = config0
    print("[gpu] config-0 block int8 weights", flush=True)
    yi, yt = run_block(device, C0, w, xi, xt, temb, cos, sin, DT.BFloat16, int8=True)
    qi, qt = oracle_block(C0, dequantized(w), xi, xt, temb, cos, sin)
    assert rel_err(yi.reshape(qi.shape), qi) <= 2e-2 and rel_err(yt.reshape(qt.shape), qt) <= 2e-2
    assert rel_err(yi.reshape(ri.shape), ri) <= 2e-2 and rel_err(yt.reshape(rt.shape), rt) <= 2e-2


def test_cfg_batch_is_two_single_runs(device):
    """A CFG batch of 2 (cond + uncond) against two batch-1 oracle runs (the
    reference's two sequential Predict calls, GenerationPipeline.cs:592-604)."""
    cfg = C0
    w, xi, xt, temb, cos, sin = block_case(cfg, 256, 64, (16, 16), batch=2, seed=5)
    yi, yt = run_block(device, cfg, w, xi, xt, temb, cos, sin, DT.BFloat16)
    for b in range(2):
        ri, rt = oracle_block(cfg, w, xi[b], xt[b], temb[b], cos, sin)
        assert rel_err(yi[b].reshape(ri.shape), ri) <= 2e-2
        assert rel_err(yt[b].reshape(rt.shape), rt) <= 2e-2


def test_padded_text_under_key_length(device):
    """A text stream padded past its real rows: the key-length mask keeps
    the padding out of every softmax (QwenImageConditioner.cs:57)."""
    cfg = mmdit.MmditConfig(width=1024, heads=8, mlp=2048, blocks=1)
    w, xi, xt, temb, cos, sin = block_case(cfg, 192, 64, (12, 16), seed=9)
    real = 192 + 40
    for compute, tol in ((DT.BFloat16, 2e-2), (DT.Float32, 1e-3)):
        yi, yt = run_block(device, cfg, w, xi, xt, temb, cos, sin, compute, key_len=real)
        ri, rt = oracle_block(cfg, w, xi, xt, temb, cos, sin, key_len=real)
        assert rel_err(yi.reshape(ri.shape), ri) <= tol
        assert rel_err(yt.reshape(rt.shape), rt) <= tol


TINY = mmdit.MmditConfig(width=256, heads=2, mlp=512, blocks=2, latent_channels=16, patch=2, text_dim=64,
                         time_dim=32)


def oracle_step(cfg, w, latent, text, t, cos, sin):
    """The step composed from oracle primitives (oracle.mmdit_step), mirroring
    the reference's Build (QwenImageDit.cs:430-505) with the dual-stream
    blocks."""
    return oracle.mmdit_step(latent, text, t, w, cfg.blocks, cfg.heads, cos, sin, cfg.patch, cfg.eps)


@pytest.mark.parametrize("compute,tol", [(DT.BFloat16, 2e-2), (DT.Float32, 1e-3)])
def test_full_step_against_oracle(device, compute, tol):
    cfg = TINY
    w = mmdit.synthetic_weights(cfg, 3, norm_spread=0.1)
    H, W, nt = 12, 16, 8
    latent = rng.normal(rng.tensor_seed(3, "latent"), (1, cfg.latent_channels, H, W))
    text = rng.normal(rng.tensor_seed(3, "text"), (1, 1, nt, cfg.text_dim))
    den = mmdit.QwenImageMmdit(device, cfg, w, H, W, nt, compute)
    out = den.Predict(HostTensor.FromFloats(latent), 500, 0.5, {"context": text}).ToFloats()
    ref = oracle_step(cfg, w, latent, text, 0.5, den.cos, den.sin)
    err = rel_err(out, ref)
    print(f"[gpu] tiny step {compute.name} rel err {err:.2e}", flush=True)
    assert out.shape == ref.shape
    assert err <= tol


def test_two_streams_match_one_stream_bit_for_bit(device, config0):
    """The text stream on the second stream changes the order of launches,
    not any arithmetic: the block's outputs equal the one-stream run's
    exactly, over several runs (the cross-stream waits and the arena reuse
    between the streams hold)."""
    w, xi, xt, temb, cos, sin, _ = config0
    one = run_block(device, C0, w, xi, xt, temb, cos, sin, DT.BFloat16, two_streams=False)
    for _ in range(3):
        two = run_block(device, C0, w, xi, xt, temb, cos, sin, DT.BFloat16, two_streams=True)
        assert np.array_equal(one[0], two[0]) and np.array_equal(one[1], two[1])
