"""Loading HuggingFace-format checkpoints (`config.json` + `model.safetensors`)
onto the HIP backend, as the reference loads them (src/arch/llm/hf.rs,
llama.rs:221-335, lfm2.rs:134-270).

The storage policy is the reference's: `KERNRT_Q8_0X4`, then `KERNRT_Q8_0`,
select the Q8 storages; otherwise a bf16 checkpoint stays bf16 and anything
else f32 (llama.rs:242-254). Each matrix then takes the form `matrix_from_raw`
(hf.rs:151-200) gives it, including its quirk: a non-bf16 file asked for Q8_0
becomes **bf16** (truncated), not Q8_0. The HIP backend holds Q8_0 and Q8_0x4
matrices only, so such a matrix is refused at upload with an error naming the
variables that select a Q8 storage. Q8 matrices are quantized on the device
from the file's f32 values or bf16 bit patterns (`kr_matrix_quantize`), with
the reference's `Matrix::from_f32_q8_0` / `Q8_0x4::from_f32` arithmetic.
"""

from __future__ import annotations

import json
import math
import os
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import safetensors
from .backends import LayerWeights, ModelWeights, SourceMatrix
from .llm import Config, Model
from .safetensors import RawTensor, SafeTensorsError

Q8_0_BLOCK = 32
Q8_0X4_ROWS = 4
STORAGES = ("f32", "bf16", "q8_0", "q8_0x4")  # hf.rs:79-86


class LoadError(Exception):
    """Errors from loading a HuggingFace-format model (hf.rs:18-41)."""


class MissingTensor(LoadError):
    def __init__(self, name: str):
        super().__init__(f"no tensor named {name!r} in the weight files")
        self.name = name


class BadConfig(LoadError):
    def __init__(self, msg: str):
        super().__init__(f"config not usable: {msg}")


def storage_from_env(bf16: bool) -> str:
    """The storage choice of `from_hf_with` (llama.rs:242-254, lfm2.rs:148-156);
    a variable counts as set whatever its value."""
    env = os.environ
    if env.get("KERNRT_Q8_0X4") is not None:
        return "q8_0x4"
    if env.get("KERNRT_Q8_0") is not None:
        return "q8_0"
    if bf16 and env.get("KERNRT_ALL_F32") is None:
        return "bf16"
    return "f32"


# ---- tensors out of the map (hf.rs:88-149) ----------------------------------

def take_raw(tensors: Dict[str, RawTensor], name: str) -> RawTensor:
    t = tensors.pop(name, None)
    if t is None:
        raise MissingTensor(name)
    return t


def take_f32(tensors: Dict[str, RawTensor], name: str) -> np.ndarray:
    return take_raw(tensors, name).widen()


def take_optional_raw(tensors: Dict[str, RawTensor], name: str) -> Optional[RawTensor]:
    return tensors.pop(name, None)


def take_optional_f32(tensors: Dict[str, RawTensor], name: str) -> Optional[np.ndarray]:
    t = tensors.pop(name, None)
    return None if t is None else t.widen()


def take_matrix_raw(tensors: Dict[str, RawTensor], name: str, storage: str) -> SourceMatrix:
    return matrix_from_raw(take_raw(tensors, name), storage)


def _bf16_truncate(values: np.ndarray) -> np.ndarray:
    # hf.rs:187-192: the top 16 bits of each f32, no rounding
    return (np.ascontiguousarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16).ravel()


def matrix_from_raw(t: RawTensor, storage: str) -> SourceMatrix:
    """The form a weight matrix takes for `storage` (hf.rs:151-200)."""
    if storage not in STORAGES:
        raise ValueError(f"unknown storage {storage!r}")
    shape = t.shape
    if len(shape) != 2:
        raise BadConfig("weight matrices must have two dimensions")
    out_dim, in_dim = shape
    aligned_q8x4 = in_dim % Q8_0_BLOCK == 0 and out_dim % Q8_0X4_ROWS == 0
    if t.dtype == "BF16":
        bits = np.asarray(t.data).ravel()
        if storage == "bf16":
            return SourceMatrix("bf16", out_dim, in_dim, bits)
        if storage == "q8_0" and in_dim % Q8_0_BLOCK == 0:
            return SourceMatrix("q8_0", out_dim, in_dim, bits)
        if storage == "q8_0x4" and aligned_q8x4:
            return SourceMatrix("q8_0x4", out_dim, in_dim, bits)
    values = t.widen().ravel()
    if storage == "f32":
        return SourceMatrix("f32", out_dim, in_dim, values)
    if storage == "q8_0x4" and aligned_q8x4:
        return SourceMatrix("q8_0x4", out_dim, in_dim, values)
    # q8_0 from a non-bf16 file, an unaligned Q8 shape, or bf16 from f32/f16:
    # narrowed to bf16 rather than widened (hf.rs:184-193)
    return SourceMatrix("bf16", out_dim, in_dim, _bf16_truncate(values))


# ---- config.json (hf.rs:202-421) ---------------------------------------------

def _read_json(path):
    try:
        with open(path, "rb") as f:
            raw = f.read()
    except OSError as e:
        raise LoadError(f"could not read the checkpoint: {e}") from e
    try:
        return json.loads(raw)
    except ValueError as e:
        raise LoadError(f"config.json does not parse: {e}") from e


def _u64(value: dict, key: str) -> Optional[int]:
    v = value.get(key) if isinstance(value, dict) else None
    if isinstance(v, bool) or not isinstance(v, int) or v < 0:
        return None
    return v


def _f64(value: dict, key: str) -> Optional[float]:
    v = value.get(key) if isinstance(value, dict) else None
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    return float(v)


def _bool(value: dict, key: str) -> Optional[bool]:
    v = value.get(key) if isinstance(value, dict) else None
    return v if isinstance(v, bool) else None


def _get(value: dict, key: str) -> int:
    v = _u64(value, key)
    if v is None:
        raise BadConfig(f"{key!r} must be present as a non-negative integer")
    return v


def _f32(x: float) -> float:
    # `as f32`: round the f64 to the nearest f32
    return float(np.float32(x))


def _check_heads(c: Config):
    # hf.rs:265-270 / 398-403; a zero head count is refused rather than divided by
    if c.n_kv_heads == 0 or c.head_dim == 0 or c.n_heads % c.n_kv_heads != 0:
        raise BadConfig("the model dimension is not a multiple of the head counts")


def parse_hf_config(path) -> Tuple[Config, bool]:
    """A Llama-family `config.json` (SmolLM2, Qwen3) and whether the weights are
    bf16 (hf.rs:202-272). Qwen3 nests the rotary base under
    `rope_parameters`; an explicit `head_dim` wins over dim / n_heads."""
    value = _read_json(path)
    n_heads = _get(value, "num_attention_heads")
    dim = _get(value, "hidden_size")
    n_kv = _u64(value, "num_key_value_heads")
    n_kv = n_heads if n_kv is None else n_kv
    theta = _f64(value, "rope_theta")
    if theta is None:
        rp = value.get("rope_parameters") if isinstance(value, dict) else None
        theta = _f64(rp, "rope_theta") if isinstance(rp, dict) else None
    head_dim = _u64(value, "head_dim")
    if head_dim is None:
        if n_heads == 0:
            raise BadConfig("the model dimension is not a multiple of the head counts")
        head_dim = dim // n_heads
    eps = _f64(value, "rms_norm_eps")
    inter = _bool(value, "rope_interleaved")
    c = Config(dim=dim, hidden_dim=_get(value, "intermediate_size"), n_layers=_get(value, "num_hidden_layers"),
               n_heads=n_heads, n_kv_heads=n_kv, vocab_size=_get(value, "vocab_size"),
               seq_len=_get(value, "max_position_embeddings"),
               rms_eps=_f32(1e-5 if eps is None else eps),
               rope_theta=_f32(10_000.0 if theta is None else theta),
               rope_interleaved=False if inter is None else inter, head_dim=head_dim)
    _check_heads(c)
    return c, value.get("torch_dtype") == "bfloat16"


def lfm2_ff_dim(block_ff_dim: int, auto_adjust: bool, multiplier: Optional[float], multiple_of: int) -> int:
    """LFM2's MLP width from its block hyperparameters (hf.rs:274-296)."""
    dim = block_ff_dim
    if auto_adjust:
        dim = dim * 2 // 3
        if multiplier is not None:
            x = multiplier * float(dim)
            dim = 0 if (math.isnan(x) or x <= 0) else int(x)  # `as usize` saturates
        if multiple_of == 0:
            raise BadConfig("block_multiple_of must be at least 1")
        dim = multiple_of * (-(-dim // multiple_of))
    return dim


def parse_lfm2_config(path) -> Tuple[Config, bool, List[bool], int]:
    """An LFM2 `config.json` (hf.rs:298-405): the config (context capped at
    8192), whether the weights are bf16, each layer's kind (True =
    attention) and the conv kernel width."""
    value = _read_json(path)
    dim = _get(value, "hidden_size")
    n_heads = _get(value, "num_attention_heads")
    n_kv = _get(value, "num_key_value_heads")
    n_layers = _get(value, "num_hidden_layers")
    idx = value.get("full_attn_idxs") if isinstance(value, dict) else None
    if isinstance(idx, list):
        full = {v for v in idx if isinstance(v, int) and not isinstance(v, bool) and v >= 0}
    else:
        full = set(range(n_layers))
    is_attn = [l in full for l in range(n_layers)]
    mult_of = _u64(value, "block_multiple_of")
    hidden = lfm2_ff_dim(_get(value, "block_ff_dim"), bool(_bool(value, "block_auto_adjust_ff_dim") or False),
                         _f64(value, "block_ffn_dim_multiplier"), 1 if mult_of is None else mult_of)
    conv_k = _u64(value, "conv_L_cache")
    eps = _f64(value, "norm_eps")
    theta = _f64(value, "rope_theta")
    if n_heads == 0:
        raise BadConfig("the model dimension is not a multiple of the head counts")
    c = Config(dim=dim, hidden_dim=hidden, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv,
               vocab_size=_get(value, "vocab_size"), seq_len=min(_get(value, "max_position_embeddings"), 8192),
               rms_eps=_f32(1e-5 if eps is None else eps),
               rope_theta=_f32(1_000_000.0 if theta is None else theta),
               rope_interleaved=False, head_dim=dim // n_heads)
    _check_heads(c)
    return c, value.get("torch_dtype") == "bfloat16", is_attn, 3 if conv_k is None else conv_k


# ---- weights (llama.rs:275-335, lfm2.rs:161-270) -------------------------------

def llama_weights(config: Config, storage: str, tensors: Dict[str, RawTensor]) -> ModelWeights:
    """`Llama::from_raw_tensors_with`'s tensor names and forms (llama.rs:275-335)."""
    emb = take_matrix_raw(tensors, "model.embed_tokens.weight", storage)
    rms_final = take_f32(tensors, "model.norm.weight")
    layers = []
    for l in range(config.n_layers):
        p = f"model.layers.{l}"
        rms_att = take_f32(tensors, f"{p}.input_layernorm.weight")
        proj = {
            "q": take_matrix_raw(tensors, f"{p}.self_attn.q_proj.weight", storage),
            "k": take_matrix_raw(tensors, f"{p}.self_attn.k_proj.weight", storage),
            "v": take_matrix_raw(tensors, f"{p}.self_attn.v_proj.weight", storage),
            "o": take_matrix_raw(tensors, f"{p}.self_attn.o_proj.weight", storage),
        }
        rms_ffn = take_f32(tensors, f"{p}.post_attention_layernorm.weight")
        proj["gate"] = take_matrix_raw(tensors, f"{p}.mlp.gate_proj.weight", storage)
        proj["down"] = take_matrix_raw(tensors, f"{p}.mlp.down_proj.weight", storage)
        proj["up"] = take_matrix_raw(tensors, f"{p}.mlp.up_proj.weight", storage)
        layers.append(LayerWeights(
            rms_att=rms_att, rms_ffn=rms_ffn, proj=proj,
            rms_q=take_optional_f32(tensors, f"{p}.self_attn.q_norm.weight"),
            rms_k=take_optional_f32(tensors, f"{p}.self_attn.k_norm.weight"), is_attention=True))
    # tied models store no lm_head
    head = take_optional_raw(tensors, "lm_head.weight")
    wcls = matrix_from_raw(head, storage) if head is not None else None
    return ModelWeights(emb, layers, rms_final, wcls)


def lfm2_weights(config: Config, is_attention: List[bool], storage: str,
                 tensors: Dict[str, RawTensor]) -> ModelWeights:
    """`Lfm2::from_raw_tensors_with`'s tensor names and forms (lfm2.rs:161-270)."""
    if len(is_attention) != config.n_layers:
        raise ValueError("layer mask must cover every layer")
    emb = take_matrix_raw(tensors, "model.embed_tokens.weight", storage)
    rms_final = take_f32(tensors, "model.embedding_norm.weight")
    layers = []
    for l, attn in enumerate(is_attention):
        p = f"model.layers.{l}"
        proj, rms_q, rms_k, kernel = {}, None, None, None
        if attn:
            proj["q"] = take_matrix_raw(tensors, f"{p}.self_attn.q_proj.weight", storage)
            proj["k"] = take_matrix_raw(tensors, f"{p}.self_attn.k_proj.weight", storage)
            proj["v"] = take_matrix_raw(tensors, f"{p}.self_attn.v_proj.weight", storage)
            # LFM2 names it out_proj where Llama says o_proj
            proj["o"] = take_matrix_raw(tensors, f"{p}.self_attn.out_proj.weight", storage)
            rms_q = take_optional_f32(tensors, f"{p}.self_attn.q_layernorm.weight")
            rms_k = take_optional_f32(tensors, f"{p}.self_attn.k_layernorm.weight")
        else:
            proj["conv_in"] = take_matrix_raw(tensors, f"{p}.conv.in_proj.weight", storage)
            proj["conv_out"] = take_matrix_raw(tensors, f"{p}.conv.out_proj.weight", storage)
            raw = take_f32(tensors, f"{p}.conv.conv.weight")  # stored [dim, 1, k]
            if raw.ndim != 3 or raw.shape[1] != 1:
                raise BadConfig(f"{p}.conv.conv.weight is {list(raw.shape)}; a depthwise kernel is [dim, 1, k]")
            kernel = np.ascontiguousarray(raw.reshape(raw.shape[0], raw.shape[2]), np.float32)
        rms_att = take_f32(tensors, f"{p}.operator_norm.weight")
        rms_ffn = take_f32(tensors, f"{p}.ffn_norm.weight")
        proj["gate"] = take_matrix_raw(tensors, f"{p}.feed_forward.w1.weight", storage)
        proj["down"] = take_matrix_raw(tensors, f"{p}.feed_forward.w2.weight", storage)
        proj["up"] = take_matrix_raw(tensors, f"{p}.feed_forward.w3.weight", storage)
        layers.append(LayerWeights(rms_att=rms_att, rms_ffn=rms_ffn, proj=proj, rms_q=rms_q, rms_k=rms_k,
                                   conv_kernel=kernel, is_attention=attn))
    head = take_optional_raw(tensors, "lm_head.weight")
    wcls = matrix_from_raw(head, storage) if head is not None else None
    return ModelWeights(emb, layers, rms_final, wcls)


def _tensors(d):
    try:
        return safetensors.load_raw(os.path.join(d, "model.safetensors"))
    except SafeTensorsError as e:
        raise LoadError(str(e)) from e
    except OSError as e:
        raise LoadError(f"could not read the checkpoint: {e}") from e


def llama_from_hf_with(d, backend, storage: Optional[str] = None) -> Model:
    """`Llama::from_hf_with` (llama.rs:236-258) over a `Hip` backend; `storage`
    overrides the environment's choice when given."""
    config, bf16 = parse_hf_config(os.path.join(d, "config.json"))
    st = storage or storage_from_env(bf16)
    return Model(config, backend, llama_weights(config, st, _tensors(d)))


def llama_from_hf(d, storage: Optional[str] = None) -> Model:
    """`Llama::from_hf` (llama.rs:227-229): the backend from KERNRT_BACKEND."""
    from .backends import from_env
    return llama_from_hf_with(d, from_env(), storage)


def lfm2_from_hf_with(d, backend, storage: Optional[str] = None) -> Model:
    """`Lfm2::from_hf_with` (lfm2.rs:142-158) over a `Hip` backend."""
    config, bf16, is_attn, _conv_k = parse_lfm2_config(os.path.join(d, "config.json"))
    st = storage or storage_from_env(bf16)
    return Model(config, backend, lfm2_weights(config, is_attn, st, _tensors(d)), lfm2=True)


def lfm2_from_hf(d, storage: Optional[str] = None) -> Model:
    """`Lfm2::from_hf` (lfm2.rs:137-139)."""
    from .backends import from_env
    return lfm2_from_hf_with(d, from_env(), storage)
