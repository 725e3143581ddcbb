"""GPU parity of real-weight loading: tensors read from a mapped safetensors
file into HBM and narrowed there, bit for bit against the stored values
narrowed on the host (nearest even); the LoRA fold on the device, bit for
bit against the oracle's restatement of LoraMerge.Merge (and the
reference's hand-worked vectors); and a Qwen-Image 2.1 denoiser built from a
checkpoint file with a LoRA, whose prediction equals, exactly, the one built
from the same weights merged by the oracle and handed over as arrays."""

import numpy as np
import pytest

import oracle
import st_files
from naivediffusion_amd import qwen, rng, sdxl
from naivediffusion_amd.lora import LoraMerge, LoraSpec
from naivediffusion_amd.safetensors import SafetensorsFile
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor, f32_to_bf16

pytestmark = pytest.mark.gpu

FLOATS = {"F32": DT.Float32, "F16": DT.Float16, "BF16": DT.BFloat16}


def say(msg):
    print(f"[gpu] {msg}", flush=True)


def narrowed_bits(values, dtype):
    """float32 values as a host tensor of dtype would hold them (nearest
    even; numpy's float16 cast, f32_to_bf16's rounding)."""
    return HostTensor.FromFloats(np.asarray(values, np.float32)).ConvertTo(dtype).Data


def awkward_values(n, seed):
    """Values that exercise the rounding: ties, subnormals of each width,
    overflow to infinity in half, signed zeros, NaN."""
    r = np.random.default_rng(seed)
    v = (r.standard_normal(n) * np.exp2(r.integers(-30, 20, n))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 1e5, 6e-8, 3e-8, 1e-40,
                        1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8], np.float32)
    v[:len(special)] = special
    return v


@pytest.mark.parametrize("stored", ["F32", "F16", "BF16"])
def test_float_tensors_are_read_and_narrowed_bit_exactly(device, tmp_path, stored):
    v = awkward_values(4099, 5)
    path = st_files.write(tmp_path / "f.safetensors", [("w", (4099,), stored, v)])
    stored_bits = st_files.encode(stored, v)
    with SafetensorsFile(path) as f:
        wide = f.Read("w").ToFloats()
        for target in (None, DT.Float32, DT.Float16, DT.BFloat16):
            say(f"read {stored} as {target.name if target else 'stored'}")
            t = f.ReadDevice("w", device, target)
            got = t.Download()
            t.Dispose()
            if target is None or target == FLOATS[stored]:
                assert got.Data.tobytes() == stored_bits
            else:
                want = HostTensor(target, (4099,), narrowed_bits(wide, target))
                assert got.DataType == target
                # NaN stays NaN (its payload is not part of the contract);
                # every other value bit for bit, signed zeros included
                nan = np.isnan(want.ToFloats())
                assert np.array_equal(np.isnan(got.ToFloats()), nan)
                assert np.array_equal(got.Data[~nan], want.Data[~nan])


def test_large_and_integer_tensors_go_through_the_staging_exactly(device, tmp_path):
    """A tensor larger than the two 32 MiB staging buffers together (three
    chunks plus a tail), an odd byte count, integer widths copied as stored,
    a 5-axis filter folded to 4 axes, and the refusals."""
    r = np.random.default_rng(9)
    big = r.standard_normal(24 * 2 ** 20 + 3).astype(np.float32)
    ints = r.integers(-2 ** 40, 2 ** 40, 1001)
    path = st_files.write(tmp_path / "big.safetensors", [
        ("big", big.shape, "F32", big), ("i64", (1001,), "I64", ints), ("u16", (7,), "U16", np.arange(7) * 9000),
        ("i32", (3, 5), "I32", np.arange(15) - 7), ("u32", (2,), "U32", [1, 2 ** 32 - 1]),
        ("conv3d", (4, 3, 2, 3, 3), "BF16", r.standard_normal(216)), ("fp8", (4,), "F8_E4M3", None)])
    with SafetensorsFile(path) as f:
        say("read a 96 MiB float32 tensor")
        t = f.ReadDevice("big", device)
        assert np.array_equal(t.Download().Data, big)
        t.Dispose()
        t = f.ReadDevice("big", device, DT.BFloat16)
        assert np.array_equal(t.Download().Data, f32_to_bf16(big))
        t.Dispose()
        for name in ("i64", "u16", "i32", "u32"):
            t = f.ReadDevice(name, device)
            assert t.Download().Data.tobytes() == f.Read(name).Data.tobytes()
            assert t.Shape == f.Read(name).Shape
            t.Dispose()
        t = f.ReadDevice("conv3d", device)
        assert t.Shape == (12, 2, 3, 3)
        assert t.Download().Data.tobytes() == f.Read("conv3d").Data.tobytes()
        t.Dispose()
        with pytest.raises(ValueError, match="only float tensors"):
            f.ReadDevice("i32", device, DT.Float32)
        with pytest.raises(NotImplementedError, match="F8_E4M3 is not supported"):
            f.ReadDevice("fp8", device)


# ---- the LoRA fold ------------------------------------------------------------------------

def fold(device, weight: HostTensor, pairs, dtype=None):
    """pairs: (down, up, scale, first) host float arrays."""
    from naivediffusion_amd.lora import Module
    w = device.Upload(weight)
    mods = [(Module(HostTensor.FromFloats(d), HostTensor.FromFloats(u), None), s, f) for d, u, s, f in pairs]
    out = LoraMerge.Merge(w, mods, dtype)
    w.Dispose()
    res = out.Download()
    out.Dispose()
    return res


def expected(weight: HostTensor, pairs, dtype):
    merged = oracle.lora_merge(weight.ToFloats(), pairs)
    return HostTensor.FromFloats(merged).ConvertTo(dtype)


def test_fold_matches_the_reference_hand_worked_vectors(device):
    """LoraFileTests.TheDeltaIsFoldedIntoTheWeightAtTheStoredWidth."""
    pair = (np.array([[1, 2, 3]], np.float32), np.array([[10], [100]], np.float32))
    w = HostTensor.FromFloats(np.array([[1, 1, 1], [2, 2, 2]], np.float32))
    out = fold(device, w, [(*pair, oracle.lora_scale(2.0, 0.5, 1), 0)])
    assert out.DataType == DT.Float32 and out.ToFloats().tolist() == [[11, 21, 31], [102, 202, 302]]
    half = fold(device, w.ConvertTo(DT.Float16), [(*pair, oracle.lora_scale(1.0, 0.5, 1), 0)])
    assert half.DataType == DT.Float16 and half.ToFloats().tolist() == [[6, 11, 16], [52, 102, 152]]
    bf = fold(device, w.ConvertTo(DT.BFloat16), [(*pair, oracle.lora_scale(1.0, 0.5, 1), 0)])
    assert bf.DataType == DT.Float16   # bfloat16 becomes half, as the reference merges it


@pytest.mark.parametrize("wdtype", [DT.Float32, DT.Float16, DT.BFloat16])
@pytest.mark.parametrize("out", [None, DT.BFloat16, DT.Float32])
def test_fold_is_bit_exact_against_the_oracle(device, wdtype, out):
    """Several pairs over overlapping and partial row ranges (the Qwen gate/up
    halves), ranks 1..7, rows not a multiple of the kernel's 16 and columns
    not of 256, zero factors, a down value that is infinite where its factor
    is zero."""
    r = np.random.default_rng(int(wdtype) * 7 + (0 if out is None else int(out) + 1))
    rows, cols = 77, 300
    w = HostTensor.FromFloats(r.standard_normal((rows, cols)).astype(np.float32)).ConvertTo(wdtype)
    pairs = []
    for first, count, rank in ((0, 77, 4), (0, 38, 7), (38, 39, 1), (10, 20, 3)):
        d = r.standard_normal((rank, cols)).astype(np.float32)
        u = r.standard_normal((count, rank)).astype(np.float32)
        u[::5, 0] = 0.0
        pairs.append((d, u, float(np.float32(r.uniform(-2, 2))), first))
    pairs[0][0][0, 3] = np.inf
    pairs[0][1][:, 0] = 0.0
    say(f"fold {wdtype.name} -> {out.name if out is not None else 'reference width'}")
    got = fold(device, w, pairs, out)
    want = expected(w, pairs, out if out is not None else (DT.Float32 if wdtype == DT.Float32 else DT.Float16))
    assert got.DataType == want.DataType
    assert np.array_equal(got.Data, want.Data)
    assert np.isfinite(got.ToFloats()).all()


def test_more_pairs_than_one_launch_and_a_model_sized_weight(device):
    """20 pairs (two launches, float32 between them) and a 3072 x 3072
    weight with two rank-32 pairs: bit exact."""
    r = np.random.default_rng(3)
    w = HostTensor.FromFloats(r.standard_normal((40, 64)).astype(np.float32)).ConvertTo(DT.Float16)
    pairs = [(r.standard_normal((2, 64)).astype(np.float32), r.standard_normal((40, 2)).astype(np.float32),
              0.1 * (i + 1), 0) for i in range(20)]
    assert np.array_equal(fold(device, w, pairs).Data, expected(w, pairs, DT.Float16).Data)
    D = 3072
    say("fold a 3072 x 3072 weight")
    w = HostTensor.FromFloats(0.02 * r.standard_normal((D, D)).astype(np.float32)).ConvertTo(DT.BFloat16)
    pairs = [(r.standard_normal((32, D)).astype(np.float32) * 0.01, r.standard_normal((D, 32)).astype(np.float32),
              0.8, 0), (r.standard_normal((32, D)).astype(np.float32) * 0.01,
                        r.standard_normal((D // 2, 32)).astype(np.float32), -0.5, D // 2)]
    assert np.array_equal(fold(device, w, pairs, DT.BFloat16).Data, expected(w, pairs, DT.BFloat16).Data)


def test_lora_merge_apply_on_device_tensors(device, tmp_path):
    """LoraMerge.Apply over a dictionary of device tensors: the SDXL layout,
    a convolution weight (rows past the first axis), the untouched weight
    left as it was."""
    r = np.random.default_rng(4)
    down = r.standard_normal((2, 4, 3, 3)).astype(np.float32)
    up = r.standard_normal((8, 2, 1, 1)).astype(np.float32)
    lora = st_files.write(tmp_path / "conv.safetensors", [
        ("lora_unet_conv_in.lora_down.weight", down.shape, "F32", down),
        ("lora_unet_conv_in.lora_up.weight", up.shape, "F16", up),
        ("lora_unet_conv_in.alpha", (), "F32", [1.0])])
    conv = HostTensor.FromFloats(r.standard_normal((8, 4, 3, 3)).astype(np.float32)).ConvertTo(DT.Float16)
    tensors = {"conv_in.weight": device.Upload(conv), "conv_out.weight": device.Upload(HostTensor.FromFloats([7.0]))}
    untouched = tensors["conv_out.weight"]
    LoraMerge.Apply(tensors, sdxl.lora_layout(), sdxl.LORA_UNET, [LoraSpec(lora, 0.75)])
    got = tensors["conv_in.weight"].Download()
    up16 = HostTensor.FromFloats(up).ConvertTo(DT.Float16).ToFloats()
    want = expected(conv, [(down.reshape(2, -1), up16.reshape(8, 2), oracle.lora_scale(0.75, 1.0, 2), 0)],
                    DT.Float16)
    assert got.Shape == (8, 4, 3, 3) and np.array_equal(got.Data, want.Data)
    assert tensors["conv_out.weight"] is untouched
    for t in tensors.values():
        t.Dispose()


# ---- a model from a checkpoint file ---------------------------------------------------------

SMALL = qwen.QwenImageConfig(width=256, heads=2, mlp=384, blocks=2, latent_channels=64, context_width=128, time_dim=64)


def qwen_file(tmp_path, w, fused: bool, prefix=""):
    tensors = []
    for k, v in w.items():
        if not fused and k.endswith(qwen.FUSED_GATE_UP):
            block = k[: -len(qwen.FUSED_GATE_UP)]
            F = v.shape[0] // 2
            tensors += [(prefix + block + qwen.GATE_PROJECTION, v[:F].shape, "BF16", v[:F]),
                        (prefix + block + qwen.UP_PROJECTION, v[F:].shape, "BF16", v[F:])]
        else:
            tensors.append((prefix + k, v.shape, "BF16", v))
    return st_files.write(tmp_path / f"qwen_{int(fused)}.safetensors", tensors)


@pytest.mark.parametrize("fused,prefix", [(True, ""), (False, "model.diffusion_model.")])
def test_qwen_denoiser_from_a_checkpoint_with_a_lora(device, tmp_path, fused, prefix):
    cfg = SMALL
    D, F = cfg.width, cfg.mlp
    w = qwen.synthetic_weights(cfg, 81, norm_spread=0.1)
    path = qwen_file(tmp_path, w, fused, prefix)
    r = np.random.default_rng(81)

    def pair(rank, rows, cols):
        return (0.05 * r.standard_normal((rank, cols))).astype(np.float32), r.standard_normal((rows, rank)).astype(
            np.float32)

    dq, uq = pair(4, D, D)          # PEFT names, an alpha: folded before the pair rotation
    dg, ug = pair(2, F, D)          # the gate half of the fused matrix
    du, uu = pair(3, F, D)          # the up half
    dp, up_ = pair(2, cfg.latent_channels, D)   # kohya names
    lora = st_files.write(tmp_path / "turbo.safetensors", [
        ("transformer.transformer_blocks.0.attn.to_q.lora_A.weight", dq.shape, "F16", dq),
        ("transformer.transformer_blocks.0.attn.to_q.lora_B.weight", uq.shape, "F16", uq),
        ("transformer.transformer_blocks.0.attn.to_q.alpha", (), "F32", [8.0]),
        ("diffusion_model.transformer_blocks.1.img_mlp.gate_layer.lora_A.weight", dg.shape, "BF16", dg),
        ("diffusion_model.transformer_blocks.1.img_mlp.gate_layer.lora_B.weight", ug.shape, "BF16", ug),
        ("transformer_blocks.1.img_mlp.proj.lora_A.weight", du.shape, "F32", du),
        ("transformer_blocks.1.img_mlp.proj.lora_B.weight", uu.shape, "F32", uu),
        ("lora_unet_proj_out.lora_down.weight", dp.shape, "F32", dp),
        ("lora_unet_proj_out.lora_up.weight", up_.shape, "F32", up_)])
    strength = 0.9

    def stored(x, dt):
        return HostTensor.FromFloats(x).ConvertTo(dt).ToFloats()

    # the oracle's merge of the same weights, narrowed to the loaded width
    merged = dict(w)
    key_q = "transformer_blocks.0.attn.to_q.weight"
    merged[key_q] = oracle.lora_merge(w[key_q], [(stored(dq, DT.Float16), stored(uq, DT.Float16),
                                                  oracle.lora_scale(strength, 8.0, 4), 0)])
    if fused:
        key_g = "transformer_blocks.1." + qwen.FUSED_GATE_UP
        merged[key_g] = oracle.lora_merge(w[key_g], [(stored(dg, DT.BFloat16), stored(ug, DT.BFloat16),
                                                      oracle.lora_scale(strength, None, 2), 0),
                                                     (du, uu, oracle.lora_scale(strength, None, 3), F)])
    merged["proj_out.weight"] = oracle.lora_merge(w["proj_out.weight"], [(dp, up_, oracle.lora_scale(strength, None, 2), 0)])
    merged = {k: stored(v, DT.BFloat16).reshape(v.shape) for k, v in merged.items()}

    H, W, n_txt, real = 8, 10, 16, 12
    latent = rng.normal(rng.tensor_seed(81, "latent"), (cfg.latent_channels, H, W))
    cond = qwen.conditioning(rng.normal(rng.tensor_seed(81, "ctx"), (real, cfg.context_width)), n_txt, H, W)
    with SafetensorsFile(path) as f:
        assert qwen.dit_prefix(f) == prefix
        say(f"qwen denoiser from a checkpoint file ({'fused' if fused else 'split'} gate/up, prefix '{prefix}')")
        loaded_cfg, weights = qwen.load_dit(f, device, [LoraSpec(lora, strength)], DT.BFloat16)
        assert loaded_cfg == cfg
        if not fused:
            # the split halves are folded one by one; the oracle does the same
            for name, (d, u, rank, dt) in {qwen.GATE_PROJECTION: (dg, ug, 2, DT.BFloat16),
                                           qwen.UP_PROJECTION: (du, uu, 3, DT.Float32)}.items():
                key = "transformer_blocks.1." + name
                half = w["transformer_blocks.1." + qwen.FUSED_GATE_UP][:F] if name == qwen.GATE_PROJECTION else \
                    w["transformer_blocks.1." + qwen.FUSED_GATE_UP][F:]
                merged_half = oracle.lora_merge(half, [(stored(d, dt), stored(u, dt),
                                                        oracle.lora_scale(strength, None, rank), 0)])
                merged[key] = stored(merged_half, DT.BFloat16).reshape(half.shape)
            g = merged.pop("transformer_blocks.1." + qwen.GATE_PROJECTION)
            u = merged.pop("transformer_blocks.1." + qwen.UP_PROJECTION)
            merged["transformer_blocks.1." + qwen.FUSED_GATE_UP] = np.concatenate([g, u], 0)
        den = qwen.QwenImageDit(device, cfg, weights, H * 16, W * 16, n_txt, DT.BFloat16)
        weights.Dispose()
    from_file = den.Predict(HostTensor.FromFloats(latent), 500, 0.45, cond).ToFloats()
    den.Dispose()
    den = qwen.QwenImageDit(device, cfg, merged, H * 16, W * 16, n_txt, DT.BFloat16)
    from_arrays = den.Predict(HostTensor.FromFloats(latent), 500, 0.45, cond).ToFloats()
    den.Dispose()
    assert np.array_equal(from_file, from_arrays)
    # the LoRA changed the prediction
    den = qwen.QwenImageDit(device, cfg, w, H * 16, W * 16, n_txt, DT.BFloat16)
    plain = den.Predict(HostTensor.FromFloats(latent), 500, 0.45, cond).ToFloats()
    den.Dispose()
    assert not np.array_equal(plain, from_file)
