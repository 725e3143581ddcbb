"""Checkpoint files and LoRAs on the CPU: the mapped reader's header checks
through the C ABI (no device needed to open, list or window a file), the
LoRA layouts, pairing and matching, and the oracle of the fold pinned to
the reference's hand-worked vectors and to what float32 arithmetic fixes."""

import os

import numpy as np
import pytest

import oracle
import st_files
from naivediffusion_amd import anima, qwen, sdxl
from naivediffusion_amd.lora import LoraFile, LoraMerge, LoraPatchSet, LoraRows, LoraSpec
from naivediffusion_amd.safetensors import InvalidDataError, IsSupportedDataType, SafetensorsFile
from naivediffusion_amd.tensors import HostDataType as DT, f32_to_bf16


# ---- the reader ------------------------------------------------------------------------

def test_a_file_written_by_the_safetensors_package_reads_back_exactly(tmp_path):
    from safetensors.numpy import save_file
    r = np.random.default_rng(0)
    tensors = {"a.weight": r.standard_normal((3, 5)).astype(np.float32),
               "b": r.standard_normal(7).astype(np.float16),
               "ints": np.arange(-4, 4, dtype=np.int64), "u": np.arange(6, dtype=np.uint16).reshape(2, 3),
               "i": np.arange(4, dtype=np.int32), "scalar": np.array(3.5, np.float32),
               "empty": np.zeros((0, 4), np.float32)}
    path = str(tmp_path / "x.safetensors")
    save_file(tensors, path, metadata={"modelspec.architecture": "test", "note": "é ✓"})
    with SafetensorsFile(path) as f:
        assert sorted(f.Keys) == sorted(tensors)
        assert f.Metadata == {"modelspec.architecture": "test", "note": "é ✓"}
        for k, v in tensors.items():
            ok, dtype, shape = f.TryGetInfo(k)
            assert ok and shape == v.shape
            t = f.Read(k)
            assert t.Shape == v.shape and np.array_equal(t.Data, v)
            assert not t.Data.flags.writeable
        assert f.TryGetInfo("missing") == (False, "", ())
        with pytest.raises(KeyError):
            f.Read("missing")
        assert set(f.ReadPrefix("a.")) == {"weight"}


def test_bfloat16_is_read_as_the_top_half_of_float32(tmp_path):
    exact = np.array([1.0, -2.5, 3.140625, 65280.0, np.inf], np.float32)
    v = np.append(exact, np.float32(1e-30))
    path = st_files.write(tmp_path / "bf.safetensors", [("w", (6,), "BF16", v)])
    with SafetensorsFile(path) as f:
        t = f.Read("w")
        assert t.DataType == DT.BFloat16 and t.Data.dtype == np.uint16
        wide = t.ToFloats()
        assert np.array_equal(wide[:5], exact)
        assert abs(wide[5] - 1e-30) <= 1e-30 * 2.0 ** -8


def test_unsupported_widths_are_listed_but_not_read(tmp_path):
    """The header of a file quantised to a width the library cannot run is
    still read (SafetensorsFile.cs:136-141); only Read refuses it."""
    path = st_files.write(tmp_path / "fp8.safetensors", [("w", (4,), "F8_E4M3", None), ("x", (2,), "F32", [1, 2])])
    with SafetensorsFile(path) as f:
        assert f.TryGetInfo("w") == (True, "F8_E4M3", (4,))
        with pytest.raises(NotImplementedError, match="F8_E4M3 is not supported"):
            f.Read("w")
        assert np.array_equal(f.Read("x").Data, [1, 2])
    assert [IsSupportedDataType(d) for d in ("F32", "F16", "BF16", "U32", "I32", "U16", "I64", "I8", "F8_E4M3")] \
        == [True] * 7 + [False, False]


def test_files_that_are_not_safetensors_are_refused_without_reading_past_the_end(tmp_path):
    """The reference's cases (CheckpointInspectorTests.cs:219-255) plus the
    JSON edges: every one is InvalidDataError, none reads outside the file."""
    whole = st_files.write(tmp_path / "whole.safetensors", [("a", (4, 4), "F32", np.ones(16)),
                                                             ("b", (8,), "F16", np.ones(8))])
    data = open(whole, "rb").read()
    cases = {
        "empty": b"\0\0",
        "random": bytes((i * 131 + 7) & 255 for i in range(4096)),
        "truncated": data[:40],
        "overrun": data[:-1],
    }
    paths = [str(tmp_path / f"{k}.safetensors") for k in cases]
    for p, b in zip(paths, cases.values()):
        open(p, "wb").write(b)
    headers = {
        "notatable": b'{"a":1}',
        "noshape": b'{"a":{"dtype":"F16","data_offsets":[0,0]}}',
        "nodtype": b'{"a":{"dtype":null,"shape":[0],"data_offsets":[0,0]}}',
        "array": b"[1,2,3]",
        "badjson": b'{"a":',
        "trailing": b'{"a":{"dtype":"F16","shape":[0],"data_offsets":[0,0]}} x',
        "negative": b'{"a":{"dtype":"F16","shape":[1],"data_offsets":[-2,0]}}',
        "backwards": b'{"a":{"dtype":"F16","shape":[1],"data_offsets":[2,0]}}',
        "fraction": b'{"a":{"dtype":"F16","shape":[1.5],"data_offsets":[0,0]}}',
        "metadata": b'{"__metadata__":[1]}',
    }
    paths += [st_files.with_header(tmp_path / f"{k}.safetensors", v) for k, v in headers.items()]
    too_long = tmp_path / "toolong.safetensors"
    too_long.write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
    paths.append(str(too_long))
    for p in paths:
        with pytest.raises(InvalidDataError):
            SafetensorsFile(p)
    # the same refusal names the reason
    with pytest.raises(InvalidDataError, match="too short"):
        SafetensorsFile(paths[0])
    with pytest.raises(InvalidDataError, match="points outside the file"):
        SafetensorsFile(paths[3])
    with pytest.raises(InvalidDataError, match="does not fit the file"):
        SafetensorsFile(paths[2])


def test_json_the_writers_produce_is_read(tmp_path):
    """Escapes, non-ASCII names, space padding (the Rust writer pads the
    header to 8 bytes), non-string metadata skipped, a name written twice
    keeping the later entry."""
    header = ('{"__metadata__":{"s":"a\\"b\\\\c\\u00e9\\ud83d\\ude00","n":3,"o":{"x":1}},'
              '"w\\u00e9":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
              '"d":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
              '"d":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}').encode() + b"   \n\t"
    path = tmp_path / "j.safetensors"
    path.write_bytes(len(header).to_bytes(8, "little") + header + np.array([1.5, 2.5], np.float32).tobytes())
    with SafetensorsFile(str(path)) as f:
        assert f.Metadata == {"s": 'a"b\\cé\U0001F600'}
        assert sorted(f.Keys) == ["d", "wé"]
        assert np.array_equal(f.Read("wé").Data, [1.5, 2.5])
        assert np.array_equal(f.Read("d").Data, [2.5])


def test_a_window_outlives_dispose_but_reads_do_not(tmp_path):
    path = st_files.write(tmp_path / "w.safetensors", [("w", (3,), "F32", [1, 2, 3])])
    f = SafetensorsFile(path)
    t = f.Read("w")
    f.Dispose()
    with pytest.raises(RuntimeError, match="disposed"):
        f.Read("w")
    assert np.array_equal(t.Data, [1, 2, 3])   # the mapping lives as long as the window


# ---- LoRA files --------------------------------------------------------------------------

SDXL_LORA = [
    ("lora_unet_input_blocks_4_1_transformer_blocks_0_attn1_to_k.lora_down.weight", (4, 320), "F16", None),
    ("lora_unet_input_blocks_4_1_transformer_blocks_0_attn1_to_k.lora_up.weight", (320, 4), "F16", None),
    ("lora_unet_input_blocks_4_1_transformer_blocks_0_attn1_to_k.alpha", (1,), "F16", None),
    ("lora_te1_text_model_encoder_layers_0_mlp_fc1.lora_down.weight", (4, 768), "F16", None),
    ("lora_te1_text_model_encoder_layers_0_mlp_fc1.lora_up.weight", (3072, 4), "F16", None),
]


def test_kohya_pairs_are_filed_by_tower_and_layer_with_their_alpha(tmp_path):
    """LoraFileTests.KohyaPairsAreFiledByTowerAndLayerWithTheirAlpha."""
    files = [t if not t[0].endswith(".alpha") else (t[0], t[1], t[2], [2.0]) for t in SDXL_LORA]
    f = LoraFile(st_files.write(tmp_path / "kohya.safetensors", files), sdxl.lora_layout())
    assert f.Name == "kohya"
    unet = f.Modules(sdxl.LORA_UNET)
    assert list(unet) == ["input_blocks_4_1_transformer_blocks_0_attn1_to_k"]
    m = unet["input_blocks_4_1_transformer_blocks_0_attn1_to_k"]
    assert m.Down.Shape == (4, 320) and m.Up.Shape == (320, 4) and m.Alpha == 2.0
    assert list(f.Modules(sdxl.LORA_TEXT_ENCODER).values())[0].Alpha is None
    assert f.Modules(sdxl.LORA_TEXT_ENCODER_2) == {}
    f.Dispose()


def test_peft_names_are_read_into_the_same_towers(tmp_path):
    """LoraFileTests.PeftNamesAreReadIntoTheSameTowers."""
    f = LoraFile(st_files.write(tmp_path / "peft.safetensors", [
        ("unet.down_blocks.1.attentions.0.transformer_blocks.0.attn1.to_k.lora_A.weight", (4, 320), "F16", None),
        ("unet.down_blocks.1.attentions.0.transformer_blocks.0.attn1.to_k.lora_B.weight", (320, 4), "F16", None),
        ("text_encoder_2.text_model.encoder.layers.0.mlp.fc1.lora_A.weight", (4, 1280), "F16", None),
        ("text_encoder_2.text_model.encoder.layers.0.mlp.fc1.lora_B.weight", (5120, 4), "F16", None),
    ]), sdxl.lora_layout())
    assert list(f.Modules(sdxl.LORA_UNET)) == ["down_blocks_1_attentions_0_transformer_blocks_0_attn1_to_k"]
    assert list(f.Modules(sdxl.LORA_TEXT_ENCODER_2)) == ["text_model_encoder_layers_0_mlp_fc1"]


def test_the_files_that_are_not_plain_loras_are_refused_with_the_reason(tmp_path):
    """LoraFileTests.TheFilesThatAreNotPlainSdxlLorasAreRefusedWithTheReason,
    plus the empty file and the metadata's own word on the architecture."""
    L = sdxl.lora_layout()
    cases = [
        ("sd15", [("lora_te_text_model_encoder_layers_0_mlp_fc1.lora_down.weight", (4, 768), "F16", None),
                  ("lora_te_text_model_encoder_layers_0_mlp_fc1.lora_up.weight", (3072, 4), "F16", None)],
         "Stable Diffusion 1.x"),
        ("dora", SDXL_LORA + [("lora_unet_input_blocks_4_1_transformer_blocks_0_attn1_to_k.dora_scale", (320,),
                               "F16", None)], "DoRA"),
        ("loha", [("lora_unet_input_blocks_4_1_transformer_blocks_0_attn1_to_k.hada_w1_a", (4, 320), "F16", None)],
         "LoHa"),
        ("half", SDXL_LORA[:1], "no up matrix"),
        ("upper", SDXL_LORA[1:2], "no down matrix"),
        ("nothing", [], "holds no tensors"),
    ]
    for name, tensors, reason in cases:
        with pytest.raises(InvalidDataError, match=reason):
            LoraFile(st_files.write(tmp_path / f"{name}.safetensors", tensors), L)
    flux = st_files.write(tmp_path / "flux.safetensors", [("double_blocks.0.img_attn.hada_w1_a", (4, 4), "F16", None)],
                          metadata={"modelspec.architecture": "flux-1-dev/lora"})
    with pytest.raises(InvalidDataError, match="says it is a flux-1-dev/lora, not for SDXL"):
        LoraFile(flux, L)


def test_qwen_and_anima_layouts_read_their_trainers_names(tmp_path):
    """QwenImageLoras.cs:19-33 and AnimaLoras.cs:14-31: kohya's lora_unet_,
    ComfyUI's diffusion_model., diffusers' transformer., DiffSynth's bare
    names (Qwen only) and the text encoders'; SDXL's towers refused."""
    def pair(stem, kind="peft", rows=8, cols=4):
        a, b = (("lora_A.weight", "lora_B.weight") if kind == "peft" else ("lora_down.weight", "lora_up.weight"))
        return [(f"{stem}.{a}", (2, cols), "F32", None), (f"{stem}.{b}", (rows, 2), "F32", None)]

    q = qwen.lora_layout()
    f = LoraFile(st_files.write(tmp_path / "q.safetensors",
                                pair("lora_unet_transformer_blocks_0_attn_to_q", "kohya")
                                + pair("diffusion_model.transformer_blocks.0.attn.to_k")
                                + pair("transformer.transformer_blocks.0.attn.to_v")
                                + pair("transformer_blocks.1.img_mlp.gate_layer")
                                + pair("text_encoders.qwen3vl_8b.transformer.model.layers.0.mlp.up_proj")), q)
    assert sorted(f.Modules(qwen.LORA_DIT)) == ["transformer_blocks_0_attn_to_k", "transformer_blocks_0_attn_to_q",
                                                 "transformer_blocks_0_attn_to_v",
                                                 "transformer_blocks_1_img_mlp_gate_layer"]
    assert list(f.Modules(qwen.LORA_TEXT_ENCODER)) == ["qwen3vl_8b_transformer_model_layers_0_mlp_up_proj"]
    for layout, word in ((q, "Qwen3-VL"), (anima.lora_layout(), "Qwen3")):
        with pytest.raises(InvalidDataError, match=f"two CLIP towers where .* has {word}"):
            LoraFile(st_files.write(tmp_path / "te1.safetensors",
                                    pair("lora_te1_text_model_encoder_layers_0_mlp_fc1", "kohya")), layout)
    # Anima has no bare names: a dotted name under no prefix is unreadable
    with pytest.raises(InvalidDataError, match="no LoRA pairs"):
        LoraFile(st_files.write(tmp_path / "bare.safetensors", pair("blocks.0.self_attn.q_proj")),
                 anima.lora_layout())


def test_matching_checks_shapes_aliases_parts_and_skips_weight_zero(tmp_path):
    """LoraPatchSet.Prepare: kohya names, aliases, row parts (the Qwen fused
    gate/up halves), the shape check and its message, the scale
    weight * alpha / rank, a file that fits nothing, weight 0 never opened."""
    layout = qwen.lora_layout()
    D, F = 8, 12
    shapes = {"transformer_blocks.0.img_mlp.gate_up.weight": (2 * F, D),
              "transformer_blocks.0.attn.to_q.weight": (D, D), "proj_out.weight": (4, D)}
    path = st_files.write(tmp_path / "parts.safetensors", [
        ("transformer_blocks.0.img_mlp.gate_layer.lora_A.weight", (3, D), "F32", np.ones((3, D))),
        ("transformer_blocks.0.img_mlp.gate_layer.lora_B.weight", (F, 3), "F32", np.ones((F, 3))),
        ("transformer_blocks.0.img_mlp.gate_layer.alpha", (), "F32", [1.5]),
        ("transformer_blocks.0.img_mlp.proj.lora_A.weight", (2, D), "F32", np.ones((2, D))),
        ("transformer_blocks.0.img_mlp.proj.lora_B.weight", (F, 2), "F32", np.ones((F, 2))),
        ("lora_unet_transformer_blocks_0_attn_to_q.lora_down.weight", (2, D), "F16", np.ones((2, D))),
        ("lora_unet_transformer_blocks_0_attn_to_q.lora_up.weight", (D, 2), "F16", np.ones((D, 2))),
    ])
    ps = LoraPatchSet.Prepare(shapes, layout, qwen.LORA_DIT, [LoraSpec(path, 0.7)],
                              parts=lambda key: qwen.fused_halves(key, shapes[key][0]))
    assert sorted(ps.Keys) == ["transformer_blocks.0.attn.to_q.weight", "transformer_blocks.0.img_mlp.gate_up.weight"]
    (g, sg, fg), (u, su, fu) = ps._patches["transformer_blocks.0.img_mlp.gate_up.weight"]
    assert (fg, fu) == (0, F)
    assert sg == oracle.lora_scale(0.7, 1.5, 3) and su == oracle.lora_scale(0.7, None, 2)
    assert sg == float(np.float32(np.float32(np.float32(0.7) * np.float32(1.5)) / np.float32(3)))
    assert not ps.Touches("proj_out.weight")
    ps.Dispose()

    bad = dict(shapes, **{"transformer_blocks.0.attn.to_q.weight": (D, D + 1)})
    with pytest.raises(InvalidDataError, match=r"is \[8, 2\] x \[2, 8\] but the model's is \[8, 9\]"):
        LoraPatchSet.Prepare(bad, layout, qwen.LORA_DIT, [LoraSpec(path, 1.0)],
                             parts=lambda key: qwen.fused_halves(key, bad[key][0]))

    elsewhere = st_files.write(tmp_path / "elsewhere.safetensors", [
        ("lora_unet_somewhere_else.lora_down.weight", (1, 3), "F32", [1, 1, 1]),
        ("lora_unet_somewhere_else.lora_up.weight", (2, 1), "F32", [1, 1])])
    with pytest.raises(InvalidDataError, match="trained for a different architecture than Qwen-Image 2.1"):
        LoraPatchSet.Prepare(shapes, layout, qwen.LORA_DIT, [LoraSpec(elsewhere, 1.0)])
    # at weight zero nothing is opened, so a file that is not there is fine
    LoraPatchSet.Prepare(shapes, layout, qwen.LORA_DIT, [LoraSpec(str(tmp_path / "gone.safetensors"), 0.0)]).Dispose()

    aliased = st_files.write(tmp_path / "aliased.safetensors", [
        ("lora_unet_input_blocks_0_0.lora_down.weight", (1, 2), "F32", [1, 1]),
        ("lora_unet_input_blocks_0_0.lora_up.weight", (1, 1), "F32", [1])])
    ps = LoraPatchSet.Prepare({"conv_in.weight": (1, 2)}, sdxl.lora_layout(), sdxl.LORA_UNET,
                              [LoraSpec(aliased, 1.0)],
                              lambda key: ["input_blocks.0.0.weight"] if key == "conv_in.weight" else [])
    assert ps.Touches("conv_in.weight")
    ps.Dispose()


def test_lora_spec_combine_replaces_the_same_file_in_place(tmp_path):
    a, b = str(tmp_path / "a.safetensors"), str(tmp_path / "b.safetensors")
    combined = LoraSpec.Combine([LoraSpec(a, 1.0), LoraSpec(b, 0.5)], [LoraSpec(os.path.join(tmp_path, ".", "a.safetensors"), 0.25)])
    assert [(os.path.basename(x.Path), x.Weight) for x in combined] == [("a.safetensors", 0.25), ("b.safetensors", 0.5)]
    open(a, "wb").write(b"x")
    stamp = LoraSpec.Stamp([LoraSpec(a, 0.8), LoraSpec(b, 0.0)])
    assert stamp == LoraSpec.Stamp([LoraSpec(a, 0.8)])
    assert stamp.startswith(os.path.abspath(a) + "|1|") and stamp.endswith("|0.8")
    assert LoraSpec.Stamp([LoraSpec(b, 0.0)]) == ""


# ---- the fold's oracle -----------------------------------------------------------------------

def test_oracle_fold_matches_the_reference_hand_worked_vectors():
    """LoraFileTests.TheDeltaIsFoldedIntoTheWeightAtTheStoredWidth: W 2x3,
    down [1 2 3], up [10 100], alpha 0.5, rank 1."""
    down, up = np.array([[1, 2, 3]], np.float32), np.array([[10], [100]], np.float32)
    w = np.array([[1, 1, 1], [2, 2, 2]], np.float32)
    out = oracle.lora_merge(w, [(down, up, oracle.lora_scale(2.0, 0.5, 1), 0)])
    assert out.tolist() == [[11, 21, 31], [102, 202, 302]]
    half = oracle.lora_merge(w, [(down, up, oracle.lora_scale(1.0, 0.5, 1), 0)])
    assert oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(half)).tolist() == [[6, 11, 16], [52, 102, 152]]


def test_oracle_fold_is_exact_where_arithmetic_fixes_it():
    """What float32 fixes: a rank-1 delta of small integers is exact; each
    product is rounded before the add (not fused); the deltas go into the
    widened row one at a time, not summed first; a zero factor is skipped
    even against an infinite down value; a part covers only its rows."""
    r = np.random.default_rng(1)
    w = r.integers(-8, 8, (6, 5)).astype(np.float32)
    down, up = r.integers(-4, 4, (1, 5)).astype(np.float32), r.integers(-4, 4, (6, 1)).astype(np.float32)
    assert np.array_equal(oracle.lora_merge(w, [(down, up, 1.0, 0)]), w + up @ down)
    e = np.float32(1 + 2.0 ** -12)
    fused = oracle.lora_merge(np.array([[-(1 + 2.0 ** -11)]], np.float32), [(np.array([[e]]), np.array([[e]]), 1.0, 0)])
    assert fused[0, 0] == 0.0   # fused would leave 2^-24
    tiny = np.full((3, 1), 2.0 ** -24, np.float32)
    one_by_one = oracle.lora_merge(np.ones((1, 1), np.float32), [(tiny, np.ones((1, 3), np.float32), 1.0, 0)])
    assert one_by_one[0, 0] == 1.0   # summing the three deltas first would round up to 1 + 2^-23
    inf = oracle.lora_merge(np.ones((2, 2), np.float32),
                            [(np.array([[np.inf, 1]], np.float32), np.array([[0], [1]], np.float32), 1.0, 0)])
    assert inf.tolist() == [[1, 1], [np.inf, 2]]
    part = oracle.lora_merge(np.zeros((4, 2), np.float32),
                             [(np.ones((1, 2), np.float32), np.array([[2], [3]], np.float32), 1.0, 2)])
    assert part.tolist() == [[0, 0], [0, 0], [2, 2], [3, 3]]
    # against float64 on a random case: the rounding is all there is between them
    w = r.standard_normal((16, 24)).astype(np.float32)
    pairs = [(r.standard_normal((4, 24)).astype(np.float32), r.standard_normal((16, 4)).astype(np.float32), 0.3, 0),
             (r.standard_normal((2, 24)).astype(np.float32), r.standard_normal((8, 2)).astype(np.float32), -1.2, 8)]
    exact = w.astype(np.float64)
    for d, u, s, f in pairs:
        exact[f:f + len(u)] += s * (u.astype(np.float64) @ d.astype(np.float64))
    assert np.max(np.abs(oracle.lora_merge(w, pairs) - exact)) < 1e-5


def test_qwen_config_is_read_from_the_shapes():
    cfg = qwen.QwenImageConfig(width=256, heads=2, mlp=384, blocks=3, latent_channels=64, context_width=96,
                               time_dim=32)
    shapes = qwen.weight_shapes(cfg)
    assert qwen.config_from_shapes(shapes) == cfg
    split = {k: v for k, v in shapes.items() if "gate_up" not in k}
    split["transformer_blocks.0.img_mlp.gate_layer.weight"] = (384, 256)
    assert qwen.config_from_shapes(split).mlp == 384
    with pytest.raises(InvalidDataError, match="rotary axes"):
        qwen.config_from_shapes(dict(shapes, **{"transformer_blocks.0.attn.norm_q.weight": (64,)}))
