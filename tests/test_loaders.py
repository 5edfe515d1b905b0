"""The checkpoint loaders on the CPU: the safetensors reader
(src/formats/safetensors.rs, its own tests at :391-537 restated), the
config.json parsers and the storage policy (src/arch/llm/hf.rs, its tests at
:361-421 and llama.rs:883-960), and which tensors the Llama / LFM2 loaders
take (llama.rs:275-335, lfm2.rs:161-270). No device is touched: the matrices
come back as `SourceMatrix` descriptions."""

import json

import numpy as np
import pytest

from kernrt_amd import hf
from kernrt_amd import safetensors as st
from helpers import lfm2_tensors, llama_tensors, st_decode, st_encode, st_image, tiny_config


def f32s(*vals):
    return np.array(vals, np.float32).tobytes()


# ---- safetensors.rs ------------------------------------------------------------

def test_roundtrip_preserves_names_shapes_and_values():
    img = st_image({"fc1.weight": ("F32", (2, 3), f32s(1, 2, 3, 4, 5, 6)),
                    "fc1.bias": ("F32", (2,), f32s(-1.5, 2.5))})
    t = st.read_from(img)
    assert sorted(t) == ["fc1.bias", "fc1.weight"]
    assert t["fc1.weight"].shape == (2, 3)
    assert t["fc1.weight"].ravel().tolist() == [1, 2, 3, 4, 5, 6]
    assert t["fc1.bias"].tolist() == [-1.5, 2.5]


def test_skips_the_metadata_entry():
    t = st.read_from(st_image({"w": ("F32", (1,), f32s(7.0))}, metadata={"format": "pt"}))
    assert list(t) == ["w"] and t["w"].tolist() == [7.0]


def test_rejects_unsupported_dtype():
    with pytest.raises(st.UnsupportedDtype) as e:
        st.read_from(st_image({"w": ("I32", (1,), f32s(0.0))}))
    assert e.value.dtype == "I32"


def test_decodes_bfloat16_weights():
    t = st.read_from(st_image({"w": ("BF16", (3,), bytes([0x80, 0x3F, 0x00, 0xC0, 0x00, 0x3F]))}))
    assert t["w"].tolist() == [1.0, -2.0, 0.5]


def test_decodes_float16_weights():
    t = st.read_from(st_image({"w": ("F16", (4,), bytes([0x00, 0x3C, 0x00, 0x38, 0x00, 0xC0, 0x00, 0x00]))}))
    assert t["w"].tolist() == [1.0, 0.5, -2.0, 0.0]


def test_float16_widening_is_exact_over_every_code():
    # safetensors.rs:363-386 is the IEEE binary16 -> binary32 conversion:
    # normals, subnormals (shifted into the implicit bit), inf and NaN payloads
    codes = np.arange(65536, dtype=np.uint16)
    got = st.read_raw_from(st_image({"w": ("F16", (65536,), codes.tobytes())}))["w"].widen()
    sign = np.where(codes >> 15, -1.0, 1.0)
    e, m = (codes >> 10) & 0x1F, codes & 0x3FF
    want = np.where(e == 0, sign * m * 2.0 ** -24, sign * (1 + m / 1024) * 2.0 ** (e.astype(np.float64) - 15))
    finite = e != 0x1F
    assert np.array_equal(got[finite].astype(np.float64), want[finite])
    inf = (e == 0x1F) & (m == 0)
    assert np.all(np.isinf(got[inf])) and np.all(np.isnan(got[(e == 0x1F) & (m != 0)]))
    # NaN payloads keep their mantissa bits, shifted up by 13
    nan_bits = got[(e == 0x1F) & (m != 0)].view(np.uint32) & 0x7FFFFF
    assert np.array_equal(nan_bits, (m[(e == 0x1F) & (m != 0)].astype(np.uint32) << 13))


def test_rejects_header_longer_than_file():
    with pytest.raises(st.HeaderTooShort):
        st.read_from((999).to_bytes(8, "little") + b"{}")
    with pytest.raises(st.HeaderTooShort):
        st.read_from(b"\x01\x02")


def _one(header: dict, data: bytes) -> bytes:
    hb = json.dumps(header).encode()
    return len(hb).to_bytes(8, "little") + hb + data


def test_rejects_offsets_that_do_not_match_shape():
    with pytest.raises(st.InvalidOffsets):
        st.read_from(_one({"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, f32s(1.0)))


def test_rejects_offsets_past_end_of_file():
    with pytest.raises(st.InvalidOffsets):
        st.read_from(_one({"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, f32s(1.0)))


def test_rejects_reversed_offsets_and_malformed_specs():
    with pytest.raises(st.InvalidOffsets):
        st.read_from(_one({"w": {"dtype": "F32", "shape": [0], "data_offsets": [4, 0]}}, f32s(1.0)))
    for spec, what in [([1], "must be a JSON object"), ({"shape": [1], "data_offsets": [0, 4]}, "lacks a string dtype"),
                       ({"dtype": "F32", "data_offsets": [0, 4]}, "lacks a shape list"),
                       ({"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}, "non-negative integer"),
                       ({"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}, "non-negative integer"),
                       ({"dtype": "F32", "shape": [1]}, "lacks a data_offsets list"),
                       ({"dtype": "F32", "shape": [1], "data_offsets": [0]}, "a start and an end")]:
        with pytest.raises(st.InvalidHeader, match=what):
            st.read_from(_one({"w": spec}, f32s(1.0)))
    with pytest.raises(st.InvalidHeader, match="must be a JSON object"):
        st.read_from(_one([1, 2], b""))


def test_rejects_invalid_json():
    with pytest.raises(st.InvalidJson):
        st.read_from(len(b"not json").to_bytes(8, "little") + b"not json")


def test_a_huge_shape_cannot_overflow_the_length_check():
    with pytest.raises(st.InvalidOffsets):
        st.read_from(_one({"w": {"dtype": "F32", "shape": [2 ** 62, 8], "data_offsets": [0, 0]}}, b""))


def test_load_maps_the_file_and_keeps_bf16_bits(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.normal(size=(6, 10)).astype(np.float32)
    enc = {"a": st_encode(a, "BF16"), "b": st_encode(a, "F32"), "c": st_encode(a, "F16")}
    p = tmp_path / "model.safetensors"
    p.write_bytes(st_image(enc))
    raw = st.load_raw(p)
    assert raw["a"].dtype == "BF16" and raw["a"].data.dtype == np.uint16
    assert np.array_equal(raw["a"].data, np.frombuffer(enc["a"][2], "<u2"))
    wide = st.load(p)
    for k in "abc":
        assert np.array_equal(wide[k], st_decode(*enc[k])), k
    assert np.array_equal(wide["b"], a)
    empty = tmp_path / "empty.safetensors"
    empty.write_bytes(b"")
    with pytest.raises(st.HeaderTooShort):
        st.load_raw(empty)


# ---- hf.rs config parsing ---------------------------------------------------------

def write_json(tmp_path, obj, name="config.json"):
    p = tmp_path / name
    p.write_text(json.dumps(obj) if not isinstance(obj, str) else obj)
    return p


SMOLLM2 = {"hidden_size": 576, "intermediate_size": 1536, "num_hidden_layers": 30, "num_attention_heads": 9,
           "num_key_value_heads": 3, "vocab_size": 49152, "max_position_embeddings": 8192,
           "rms_norm_eps": 1e-05, "rope_theta": 100000.0, "rope_interleaved": False, "torch_dtype": "bfloat16"}


def test_parses_a_typical_hf_config(tmp_path):
    c, bf16 = hf.parse_hf_config(write_json(tmp_path, SMOLLM2))
    assert (c.dim, c.n_layers, c.n_heads, c.n_kv_heads) == (576, 30, 9, 3)
    assert (c.head_dim, c.kv_dim, c.kv_mul) == (64, 192, 3)
    assert c.rope_theta == 100000.0 and not c.rope_interleaved and bf16
    assert c.rms_eps == float(np.float32(1e-5))


def test_parses_a_config_with_an_independent_head_dim(tmp_path):
    c, bf16 = hf.parse_hf_config(write_json(tmp_path, {
        "hidden_size": 1024, "intermediate_size": 3072, "num_hidden_layers": 28, "num_attention_heads": 16,
        "num_key_value_heads": 8, "vocab_size": 151936, "max_position_embeddings": 40960,
        "rms_norm_eps": 1e-06, "rope_theta": 1000000.0, "head_dim": 128, "torch_dtype": "bfloat16"}))
    assert (c.head_dim, c.q_dim, c.kv_dim, c.kv_mul) == (128, 2048, 1024, 2) and bf16


def test_defaults_head_dim_and_optional_fields(tmp_path):
    cfg = {k: v for k, v in SMOLLM2.items() if k not in ("rms_norm_eps", "rope_theta", "rope_interleaved",
                                                          "torch_dtype", "num_key_value_heads")}
    c, bf16 = hf.parse_hf_config(write_json(tmp_path, cfg))
    assert (c.head_dim, c.q_dim, c.kv_dim) == (64, 576, 576)  # n_kv_heads defaults to n_heads
    assert c.rope_theta == 10000.0 and c.rms_eps == float(np.float32(1e-5)) and not bf16


def test_rope_parameters_give_the_qwen3_rotary_base(tmp_path):
    cfg = dict(SMOLLM2)
    del cfg["rope_theta"]
    cfg["rope_parameters"] = {"rope_theta": 1000000.0, "rope_type": "default"}
    c, _ = hf.parse_hf_config(write_json(tmp_path, cfg))
    assert c.rope_theta == 1000000.0


def test_config_errors(tmp_path):
    cfg = dict(SMOLLM2)
    del cfg["vocab_size"]
    with pytest.raises(hf.BadConfig, match="vocab_size"):
        hf.parse_hf_config(write_json(tmp_path, cfg))
    cfg = dict(SMOLLM2, hidden_size=576.0)
    with pytest.raises(hf.BadConfig, match="hidden_size"):
        hf.parse_hf_config(write_json(tmp_path, cfg))
    with pytest.raises(hf.BadConfig, match="multiple of the head counts"):
        hf.parse_hf_config(write_json(tmp_path, dict(SMOLLM2, num_key_value_heads=4)))
    with pytest.raises(hf.LoadError, match="config.json does not parse"):
        hf.parse_hf_config(write_json(tmp_path, "{not json"))
    with pytest.raises(hf.LoadError, match="could not read the checkpoint"):
        hf.parse_hf_config(tmp_path / "absent.json")


def test_ff_dim_matches_the_checkpoint_shapes():
    assert hf.lfm2_ff_dim(6656, True, 1.0, 256) == 4608   # 350M
    assert hf.lfm2_ff_dim(10240, True, 1.0, 256) == 6912  # 700M
    assert hf.lfm2_ff_dim(12288, True, 1.0, 256) == 8192  # 1.2B
    assert hf.lfm2_ff_dim(4096, False, None, 256) == 4096
    # the 2/3 shrink is integer division, the multiplier truncates, then round up
    assert hf.lfm2_ff_dim(100, True, 1.5, 8) == 104       # 66 -> 99 -> 104
    assert hf.lfm2_ff_dim(100, True, None, 1) == 66


LFM2 = {"hidden_size": 1024, "block_ff_dim": 6656, "block_auto_adjust_ff_dim": True,
        "block_ffn_dim_multiplier": 1.0, "block_multiple_of": 256, "num_hidden_layers": 16,
        "num_attention_heads": 16, "num_key_value_heads": 8, "vocab_size": 65536,
        "max_position_embeddings": 128000, "norm_eps": 1e-05, "rope_theta": 1000000.0,
        "conv_L_cache": 3, "torch_dtype": "bfloat16", "full_attn_idxs": [2, 5, 8, 10, 12, 14]}


def test_parses_an_lfm2_config_with_a_layer_mask_and_a_cap(tmp_path):
    c, bf16, is_attn, conv_k = hf.parse_lfm2_config(write_json(tmp_path, LFM2))
    assert (c.dim, c.hidden_dim, c.n_layers, c.seq_len) == (1024, 4608, 16, 8192)
    assert (c.head_dim, c.kv_dim) == (64, 512)
    assert not c.rope_interleaved and c.rope_theta == 1000000.0 and bf16 and conv_k == 3
    assert [l for l, a in enumerate(is_attn) if a] == [2, 5, 8, 10, 12, 14]
    cfg = {k: v for k, v in LFM2.items() if k not in ("full_attn_idxs", "conv_L_cache", "norm_eps",
                                                      "rope_theta", "block_multiple_of")}
    c, _, is_attn, conv_k = hf.parse_lfm2_config(write_json(tmp_path, cfg))
    assert all(is_attn) and conv_k == 3 and c.rope_theta == 1000000.0
    assert c.hidden_dim == 4437  # 6656 * 2 // 3, multiple of 1


# ---- storage policy and matrix forms (hf.rs:151-200, llama.rs:242-254) ---------------------

def test_storage_follows_the_environment(monkeypatch):
    for v in ("KERNRT_Q8_0X4", "KERNRT_Q8_0", "KERNRT_ALL_F32"):
        monkeypatch.delenv(v, raising=False)
    assert hf.storage_from_env(True) == "bf16" and hf.storage_from_env(False) == "f32"
    monkeypatch.setenv("KERNRT_ALL_F32", "")
    assert hf.storage_from_env(True) == "f32"
    monkeypatch.setenv("KERNRT_Q8_0", "0")  # set at all counts, as var_os().is_some()
    assert hf.storage_from_env(True) == "q8_0"
    monkeypatch.setenv("KERNRT_Q8_0X4", "1")
    assert hf.storage_from_env(False) == "q8_0x4"


def raw(dtype, a):
    return st.read_raw_from(st_image({"w": st_encode(a, dtype)}))["w"]


def test_matrix_forms_follow_matrix_from_raw():
    rng = np.random.default_rng(1)
    a = rng.normal(size=(8, 64)).astype(np.float32)
    bf = raw("BF16", a)
    m = hf.matrix_from_raw(bf, "bf16")
    assert m.kind == "bf16" and np.array_equal(m.values, bf.data)
    m = hf.matrix_from_raw(bf, "q8_0")
    assert m.kind == "q8_0" and m.values.dtype == np.uint16 and np.array_equal(m.values, bf.data)
    m = hf.matrix_from_raw(bf, "q8_0x4")
    assert m.kind == "q8_0x4" and np.array_equal(m.values, bf.data)
    m = hf.matrix_from_raw(bf, "f32")
    assert m.kind == "f32" and np.array_equal(m.values, bf.widen().ravel())
    f = raw("F32", a)
    assert hf.matrix_from_raw(f, "f32").kind == "f32"
    m = hf.matrix_from_raw(f, "q8_0x4")
    assert m.kind == "q8_0x4" and m.values.dtype == np.float32 and np.array_equal(m.values, a.ravel())
    m = hf.matrix_from_raw(raw("F16", a), "q8_0x4")
    assert m.kind == "q8_0x4" and np.array_equal(m.values, a.astype(np.float16).astype(np.float32).ravel())


def test_an_f32_file_asked_for_q8_0_becomes_truncated_bf16():
    # hf.rs:173-193: the quirk -- not Q8_0, and narrowed by truncation, not rounding
    # 1 + 2^-8 + 2^-9 is 0x3F80C000: bf16 rounding would give 0x3F81 (1.0078125),
    # truncation keeps 0x3F80 (1.0)
    x = np.full((4, 32), 1.0 + 2.0 ** -8 + 2.0 ** -9, np.float32)
    m = hf.matrix_from_raw(raw("F32", x), "q8_0")
    assert m.kind == "bf16" and m.values.dtype == np.uint16
    assert np.all(m.values == 0x3F80)


def test_unaligned_shapes_narrow_to_bf16():
    rng = np.random.default_rng(2)
    a = rng.normal(size=(6, 48)).astype(np.float32)  # in_dim not a multiple of 32
    bf = raw("BF16", a)
    for s in ("q8_0", "q8_0x4"):
        m = hf.matrix_from_raw(bf, s)
        assert m.kind == "bf16" and np.array_equal(m.values, bf.data), s
    b = rng.normal(size=(6, 64)).astype(np.float32)  # out_dim not a multiple of 4
    assert hf.matrix_from_raw(raw("F32", b), "q8_0x4").kind == "bf16"
    assert hf.matrix_from_raw(raw("BF16", b), "q8_0").kind == "q8_0"
    with pytest.raises(hf.BadConfig, match="two dimensions"):
        hf.matrix_from_raw(raw("F32", a.ravel()), "q8_0")


# ---- which tensors the loaders take -------------------------------------------------

@pytest.mark.parametrize("tied", [True, False])
def test_llama_weights_take_the_hf_names(tied):
    c = tiny_config()
    enc = llama_tensors(c, tied=tied, qk_norm=True)
    tensors = st.read_raw_from(st_image(enc))
    w = hf.llama_weights(c, "q8_0x4", tensors)
    assert list(tensors) == ["model.rotary_emb.inv_freq"]  # every model tensor taken
    assert w.token_embedding.kind == "q8_0x4" and (w.token_embedding.out_dim, w.token_embedding.in_dim) == (96, 64)
    assert (w.wcls is None) == tied
    l1 = w.layers[1]
    assert sorted(l1.proj) == sorted(["q", "k", "v", "o", "gate", "down", "up"])
    assert (l1.proj["k"].out_dim, l1.proj["o"].in_dim, l1.proj["down"].in_dim) == (32, 64, 128)
    assert np.array_equal(l1.proj["gate"].values,
                          np.frombuffer(enc["model.layers.1.mlp.gate_proj.weight"][2], "<u2"))
    assert l1.rms_q is not None and l1.rms_q.shape == (16,)
    assert np.array_equal(w.rms_final, st_decode(*enc["model.norm.weight"]))


def test_llama_weights_name_the_missing_tensor():
    c = tiny_config()
    with pytest.raises(hf.MissingTensor, match="model.layers.1.mlp.up_proj.weight"):
        hf.llama_weights(c, "q8_0", st.read_raw_from(st_image(llama_tensors(c, drop="model.layers.1.mlp.up_proj.weight"))))


def test_lfm2_weights_take_the_hf_names_and_reshape_the_conv_kernel():
    c = tiny_config(n_layers=3)
    mask = [False, True, False]
    enc = lfm2_tensors(c, mask)
    tensors = st.read_raw_from(st_image(enc))
    w = hf.lfm2_weights(c, mask, "q8_0x4", tensors)
    assert not tensors
    assert [l.is_attention for l in w.layers] == mask
    assert sorted(w.layers[0].proj) == sorted(["conv_in", "conv_out", "gate", "down", "up"])
    assert w.layers[0].conv_kernel.shape == (64, 3)
    assert np.array_equal(w.layers[0].conv_kernel,
                          st_decode(*enc["model.layers.0.conv.conv.weight"]).reshape(64, 3))
    assert w.layers[1].rms_q is not None and w.layers[0].rms_q is None
    assert w.wcls is None
    with pytest.raises(hf.BadConfig, match=r"a depthwise kernel is \[dim, 1, k\]"):
        hf.lfm2_weights(c, mask, "q8_0x4", st.read_raw_from(st_image(lfm2_tensors(c, mask, conv_shape=(64, 3)))))
