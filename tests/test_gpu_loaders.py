"""Checkpoints from disk onto the device: `kr_matrix_quantize` against the
oracle's `Matrix::from_f32_q8_0` / `Q8_0x4::from_f32` restatement, and whole
HuggingFace-format directories (config.json + model.safetensors, written here
with random weights: there are no real checkpoints offline) loaded by
`kernrt_amd.hf` and run against the oracle model built from the same file's
values. Logits are compared as raw bits."""

import json

import numpy as np
import pytest

import kernrt_amd as K
import oracle as O
from kernrt_amd import hf
from helpers import assert_bits_equal, lfm2_tensors, llama_tensors, st_decode, st_encode, st_image, tiny_config

pytestmark = pytest.mark.gpu


def special_rows(rng, n, k):
    a = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
    a[0, :32] = 0.0                                    # an all-zero block: scale 0
    a[1, 32:64] = np.linspace(-1, 1, 32)               # exact halves after scaling
    a[2, 5] = np.float32(3e38)                         # a huge element
    a[3, :32] = np.float32(1e-40)                      # subnormal block
    a[-1, -32:] = -a[-1, -32:] * 1000                  # a loud last block
    return a


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("src", ["F32", "BF16"])
@pytest.mark.parametrize("shape", [(8, 64), (96, 960), (2052, 1536), (16384, 2048)])
def test_device_quantization_matches_the_reference_quantizer(storage, src, shape):
    # (16384, 2048) f32 is 128 MiB of source: two staging chunks
    n, k = shape
    rng = np.random.default_rng(n + k)
    a = special_rows(rng, n, k)
    dtype, _, payload = st_encode(a, src)
    values = st_decode(dtype, shape, payload)          # what the file holds, widened
    src_arr = np.frombuffer(payload, "<u2" if src == "BF16" else "<f4")
    hip = K.open("hip")
    h = hip.upload_matrix(K.backends.SourceMatrix(storage, n, k, src_arr))
    q, s = hip.read_matrix(h, storage, n, k)
    om = O.Matrix(values, storage)
    if storage == "q8_0":
        oq, os_ = om.q8_0_data()
        assert np.array_equal(q.ravel(), np.asarray(oq).ravel())
        assert np.array_equal(s.ravel().view(np.uint32), np.asarray(os_, np.float32).ravel().view(np.uint32))
    else:
        assert np.array_equal(K.backends.q8_0x4_records(q, s), np.asarray(om.q8_0x4_blocks()).ravel())
    hip.close()


def write_dir(tmp_path, config_json, tensors):
    (tmp_path / "config.json").write_text(json.dumps(config_json))
    (tmp_path / "model.safetensors").write_bytes(st_image(tensors))
    return tmp_path


def hf_json(c, **extra):
    j = {"hidden_size": c.dim, "intermediate_size": c.hidden_dim, "num_hidden_layers": c.n_layers,
         "num_attention_heads": c.n_heads, "num_key_value_heads": c.n_kv_heads, "vocab_size": c.vocab_size,
         "max_position_embeddings": c.seq_len, "rms_norm_eps": 1e-5, "rope_theta": c.rope_theta,
         "torch_dtype": "bfloat16"}
    j.update(extra)
    return j


def oracle_config(c):
    return O.Config(c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len,
                    c.rms_eps, c.rope_theta, c.rope_interleaved, c.head_dim)


def oracle_llama(c, enc, storage):
    """The reference's loader on the same file: every matrix widened to f32
    and quantized by `Matrix::from_f32_*`, norms widened."""
    def v(name):
        return st_decode(*enc[name])

    w = O.Weights(c.n_layers)
    for l in range(c.n_layers):
        p = f"model.layers.{l}"
        for key, name in [("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                          ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("down", "mlp.down_proj"),
                          ("up", "mlp.up_proj")]:
            w.set_proj(l, key, O.Matrix(v(f"{p}.{name}.weight"), storage))
        w.set_norm(l, "att", v(f"{p}.input_layernorm.weight"))
        w.set_norm(l, "ffn", v(f"{p}.post_attention_layernorm.weight"))
        if f"{p}.self_attn.q_norm.weight" in enc:
            w.set_norm(l, "q", v(f"{p}.self_attn.q_norm.weight"))
            w.set_norm(l, "k", v(f"{p}.self_attn.k_norm.weight"))
    w.set_embedding(O.Matrix(v("model.embed_tokens.weight"), storage))
    w.set_final_norm(v("model.norm.weight"))
    w.set_classifier(O.Matrix(v("lm_head.weight"), storage) if "lm_head.weight" in enc else None)
    return w


def oracle_lfm2(c, mask, enc, storage):
    def v(name):
        return st_decode(*enc[name])

    w = O.Weights(c.n_layers)
    for l, attn in enumerate(mask):
        p = f"model.layers.{l}"
        if attn:
            for key, name in [("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "out_proj")]:
                w.set_proj(l, key, O.Matrix(v(f"{p}.self_attn.{name}.weight"), storage))
            w.set_norm(l, "q", v(f"{p}.self_attn.q_layernorm.weight"))
            w.set_norm(l, "k", v(f"{p}.self_attn.k_layernorm.weight"))
        else:
            w.set_proj(l, "conv_in", O.Matrix(v(f"{p}.conv.in_proj.weight"), storage))
            w.set_proj(l, "conv_out", O.Matrix(v(f"{p}.conv.out_proj.weight"), storage))
            kern = v(f"{p}.conv.conv.weight")
            w.set_conv(l, kern.reshape(kern.shape[0], kern.shape[2]))
        w.set_norm(l, "att", v(f"{p}.operator_norm.weight"))
        w.set_norm(l, "ffn", v(f"{p}.ffn_norm.weight"))
        for key, name in [("gate", "w1"), ("down", "w2"), ("up", "w3")]:
            w.set_proj(l, key, O.Matrix(v(f"{p}.feed_forward.{name}.weight"), storage))
    w.set_embedding(O.Matrix(v("model.embed_tokens.weight"), storage))
    w.set_final_norm(v("model.embedding_norm.weight"))
    w.set_classifier(None)
    return w


PROMPT = [5, 11, 2, 30, 7, 7, 19, 1, 24, 60, 3]


def check_model(gpu, cpu, what):
    assert_bits_equal(gpu.prefill(PROMPT, 0), cpu.prefill(PROMPT, 0), f"{what}: prefill")
    for i, tok in enumerate([4, 90, 17]):
        pos = len(PROMPT) + i
        assert_bits_equal(gpu.forward(tok, pos), cpu.forward(tok, pos), f"{what}: decode pos {pos}")


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_smollm2_style_directory_loads_bitwise(tmp_path, storage):
    c = tiny_config()
    enc = llama_tensors(c, tied=True, dtype="BF16")
    d = write_dir(tmp_path, hf_json(c, rope_interleaved=False), enc)
    gpu = hf.llama_from_hf_with(d, K.open("hip"), storage)
    assert gpu.storage() == storage
    cpu = O.Model(oracle_config(c), oracle_llama(c, enc, storage), "cpu")
    check_model(gpu, cpu, f"smollm2-style {storage}")


def test_qwen3_style_directory_with_head_dim_qk_norm_and_lm_head(tmp_path):
    # head_dim 32 with dim 64 and 4 heads: q is twice as wide as the model;
    # the rotary base sits under rope_parameters; an untied lm_head; f16 file
    c = tiny_config(head_dim=32, rope_theta=1_000_000.0)
    enc = llama_tensors(c, tied=False, qk_norm=True, dtype="F16", seed=9)
    j = hf_json(c, head_dim=32, torch_dtype="float16")
    del j["rope_theta"]
    j["rope_parameters"] = {"rope_theta": 1_000_000.0, "rope_type": "default"}
    d = write_dir(tmp_path, j, enc)
    gpu = hf.llama_from_hf_with(d, K.open("hip"), "q8_0x4")
    cpu = O.Model(oracle_config(c), oracle_llama(c, enc, "q8_0x4"), "cpu")
    check_model(gpu, cpu, "qwen3-style")


def test_lfm2_directory_loads_bitwise(tmp_path):
    c = tiny_config(n_layers=3, rope_theta=1_000_000.0)
    mask = [False, True, False]
    enc = lfm2_tensors(c, mask, dtype="F32")
    j = {"hidden_size": c.dim, "block_ff_dim": c.hidden_dim, "block_auto_adjust_ff_dim": False,
         "num_hidden_layers": c.n_layers, "num_attention_heads": c.n_heads, "num_key_value_heads": c.n_kv_heads,
         "vocab_size": c.vocab_size, "max_position_embeddings": c.seq_len, "norm_eps": 1e-5,
         "rope_theta": 1_000_000.0, "conv_L_cache": 3, "torch_dtype": "float32", "full_attn_idxs": [1]}
    d = write_dir(tmp_path, j, enc)
    gpu = hf.lfm2_from_hf_with(d, K.open("hip"), "q8_0x4")
    cpu = O.Model(oracle_config(c), oracle_lfm2(c, mask, enc, "q8_0x4"), "cpu", lfm2=True)
    check_model(gpu, cpu, "lfm2")


def test_an_f32_checkpoint_asked_for_q8_0_is_refused_as_bf16(tmp_path, monkeypatch):
    # hf.rs:173-193 turns it into bf16, which this backend does not hold
    for v in ("KERNRT_Q8_0X4", "KERNRT_Q8_0", "KERNRT_ALL_F32"):
        monkeypatch.delenv(v, raising=False)
    c = tiny_config()
    d = write_dir(tmp_path, hf_json(c, torch_dtype="float32"), llama_tensors(c, dtype="F32"))
    with pytest.raises(RuntimeError, match="not bf16.*KERNRT_Q8_0"):
        hf.llama_from_hf_with(d, K.open("hip"), "q8_0")
    with pytest.raises(RuntimeError, match="not f32"):
        hf.llama_from_hf_with(d, K.open("hip"))  # an f32 file with no Q8 variable stays f32
    # a bf16 checkpoint without a Q8 variable stays bf16 (llama.rs:250-251): refused too
    d2 = tmp_path / "bf16"
    d2.mkdir()
    write_dir(d2, hf_json(c), llama_tensors(c, dtype="BF16"))
    with pytest.raises(RuntimeError, match="not bf16"):
        hf.llama_from_hf_with(d2, K.open("hip"))


def test_the_environment_selects_q8_0x4(tmp_path, monkeypatch):
    c = tiny_config()
    enc = llama_tensors(c, dtype="BF16", seed=12)
    d = write_dir(tmp_path, hf_json(c), enc)
    monkeypatch.setenv("KERNRT_Q8_0X4", "1")
    monkeypatch.setenv("KERNRT_BACKEND", "hip")
    gpu = hf.llama_from_hf(d)
    assert gpu.storage() == "q8_0x4"
    cpu = O.Model(oracle_config(c), oracle_llama(c, enc, "q8_0x4"), "cpu")
    assert_bits_equal(gpu.forward(3, 0), cpu.forward(3, 0), "env q8_0x4")
