"""Shared test plumbing: hand the oracle's weights to the HIP backend.

The same quantized bytes go to both sides: the oracle builds each `Matrix`
exactly as the reference loader does (quant.rs:544-557, 124-164), and the
HIP backend receives those bytes through its C ABI.
"""

import numpy as np

import kernrt_amd as K
import oracle as O


def product_matrix(m: "O.Matrix") -> K.Q8Matrix:
    if m.storage == "q8_0":
        q, s = m.q8_0_data()
        return K.Q8Matrix("q8_0", m.out_dim, m.in_dim, quants=q, scales=s)
    if m.storage == "q8_0x4":
        return K.Q8Matrix("q8_0x4", m.out_dim, m.in_dim, blocks=m.q8_0x4_blocks())
    raise ValueError(f"the hip backend takes Q8 storages, not {m.storage}")


def product_weights(w: "O.Weights") -> K.ModelWeights:
    layers = []
    for l, d in enumerate(w.layers):
        proj = {k: product_matrix(v) for k, v in d.items() if k in K.backends.PROJ_INDEX}
        layers.append(K.LayerWeights(
            rms_att=d["norm_att"], rms_ffn=d["norm_ffn"], proj=proj,
            rms_q=d.get("norm_q"), rms_k=d.get("norm_k"), conv_kernel=d.get("conv_kernel"),
            is_attention=w.is_attention[l]))
    cls = product_matrix(w.classifier) if w.classifier is not None else None
    return K.ModelWeights(product_matrix(w.embedding), layers, w.final_norm, cls)


def product_config(c: "O.Config") -> K.Config:
    return K.Config(c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len,
                    c.rms_eps, c.rope_theta, c.rope_interleaved, c.head_dim)


def gpu_model(c: "O.Config", w: "O.Weights", lfm2: bool = False):
    """A kernrt_amd model over a fresh HIP backend, with the oracle's weights."""
    hip = K.open("hip")
    return K.Model(product_config(c), hip, product_weights(w), lfm2=lfm2)


def gaussian_weights(c: "O.Config", storage: str, seed: int, lfm2_mask=None, tied: bool = True,
                     qk_norm: bool = False, norms: str = "ones"):
    """N(0, 0.02) weights (the benchmark recipe). Norm weights are 1.0
    (norms="ones") or U(0.5, 1.5) (norms="uniform"); with qk_norm the
    attention layers get per-head q and k norm weights (Qwen3, LFM2)."""
    rng = np.random.default_rng(seed)
    dim, hidden = c.dim, c.hidden_dim

    def mat(rows, cols):
        return O.Matrix(rng.normal(0.0, 0.02, size=(rows, cols)).astype(np.float32), storage)

    def norm(n):
        if norms == "ones":
            return np.ones(n, np.float32)
        return rng.uniform(0.5, 1.5, size=n).astype(np.float32)

    w = O.Weights(c.n_layers)
    mask = lfm2_mask or [True] * c.n_layers
    for l in range(c.n_layers):
        if mask[l]:
            w.set_proj(l, "q", mat(c.q_dim, dim))
            w.set_proj(l, "k", mat(c.kv_dim, dim))
            w.set_proj(l, "v", mat(c.kv_dim, dim))
            w.set_proj(l, "o", mat(dim, c.q_dim))
            if qk_norm:
                w.set_norm(l, "q", norm(c.head_dim))
                w.set_norm(l, "k", norm(c.head_dim))
        else:
            w.set_proj(l, "conv_in", mat(3 * dim, dim))
            w.set_proj(l, "conv_out", mat(dim, dim))
            w.set_conv(l, rng.normal(0.0, 0.2, size=(dim, 3)).astype(np.float32))
        w.set_norm(l, "att", norm(dim))
        w.set_norm(l, "ffn", norm(dim))
        w.set_proj(l, "gate", mat(hidden, dim))
        w.set_proj(l, "down", mat(dim, hidden))
        w.set_proj(l, "up", mat(hidden, dim))
    w.set_embedding(mat(c.vocab_size, dim))
    w.set_final_norm(norm(dim))
    w.set_classifier(None if tied else mat(c.vocab_size, dim))
    return w


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    g, w = bits(got), bits(want)
    if not np.array_equal(g, w):
        bad = np.nonzero(g != w)[0]
        i = bad[0]
        gf, wf = np.asarray(got, np.float32).ravel(), np.asarray(want, np.float32).ravel()
        raise AssertionError(f"{what}: {bad.size} of {g.size} values differ; first at {i}: "
                             f"got {gf[i]!r} want {wf[i]!r}")


# ---- checkpoint files for the loader tests ------------------------------------

def st_image(tensors, metadata=None) -> bytes:
    """A safetensors byte image: `tensors` maps name -> (dtype, shape, payload
    bytes), laid out in order with 8-byte aligned data offsets."""
    import json
    header, data = {}, bytearray()
    for name, (dtype, shape, payload) in tensors.items():
        start = len(data)
        data += payload
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [start, len(data)]}
        data += b"\0" * (-len(data) % 8)
    if metadata is not None:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    hb += b" " * (-len(hb) % 8)
    return len(hb).to_bytes(8, "little") + hb + bytes(data)


def st_encode(a: np.ndarray, dtype: str):
    """(dtype, shape, payload) of an f32 array stored as F32, BF16 (rounded to
    nearest even, as torch does) or F16."""
    a = np.ascontiguousarray(a, np.float32)
    if dtype == "F32":
        return "F32", a.shape, a.tobytes()
    if dtype == "F16":
        return "F16", a.shape, a.astype("<f2").tobytes()
    u = a.view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return "BF16", a.shape, b.tobytes()


def st_decode(dtype: str, shape, payload: bytes) -> np.ndarray:
    """The f32 values a loader reads back from st_encode's output."""
    if dtype == "F32":
        return np.frombuffer(payload, "<f4").reshape(shape).copy()
    if dtype == "F16":
        return np.frombuffer(payload, "<f2").astype(np.float32).reshape(shape)
    b = np.frombuffer(payload, "<u2").astype(np.uint32) << 16
    return b.view(np.float32).reshape(shape)


def llama_tensors(c, tied=True, qk_norm=False, dtype="BF16", seed=3, drop=None):
    rng = np.random.default_rng(seed)
    t = {}

    def put(name, shape, scale=0.02):
        t[name] = st_encode(rng.normal(0, scale, size=shape).astype(np.float32), dtype)

    put("model.embed_tokens.weight", (c.vocab_size, c.dim))
    put("model.norm.weight", (c.dim,), 1.0)
    for l in range(c.n_layers):
        p = f"model.layers.{l}"
        put(f"{p}.input_layernorm.weight", (c.dim,), 1.0)
        put(f"{p}.post_attention_layernorm.weight", (c.dim,), 1.0)
        put(f"{p}.self_attn.q_proj.weight", (c.q_dim, c.dim))
        put(f"{p}.self_attn.k_proj.weight", (c.kv_dim, c.dim))
        put(f"{p}.self_attn.v_proj.weight", (c.kv_dim, c.dim))
        put(f"{p}.self_attn.o_proj.weight", (c.dim, c.q_dim))
        put(f"{p}.mlp.gate_proj.weight", (c.hidden_dim, c.dim))
        put(f"{p}.mlp.down_proj.weight", (c.dim, c.hidden_dim))
        put(f"{p}.mlp.up_proj.weight", (c.hidden_dim, c.dim))
        if qk_norm:
            put(f"{p}.self_attn.q_norm.weight", (c.head_dim,), 1.0)
            put(f"{p}.self_attn.k_norm.weight", (c.head_dim,), 1.0)
    if not tied:
        put("lm_head.weight", (c.vocab_size, c.dim))
    t["model.rotary_emb.inv_freq"] = st_encode(np.ones(4, np.float32), "F32")  # ignored, as the reference does
    if drop:
        del t[drop]
    return t


def tiny_config(**kw):
    from kernrt_amd.llm import Config
    base = dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, seq_len=64,
                rms_eps=1e-5, rope_theta=10000.0, rope_interleaved=False, head_dim=16)
    base.update(kw)
    return Config(**base)


def lfm2_tensors(c, is_attn, dtype="F32", seed=4, conv_shape=None, k=3):
    rng = np.random.default_rng(seed)
    t = {}

    def put(name, shape, scale=0.02):
        t[name] = st_encode(rng.normal(0, scale, size=shape).astype(np.float32), dtype)

    put("model.embed_tokens.weight", (c.vocab_size, c.dim))
    put("model.embedding_norm.weight", (c.dim,), 1.0)
    for l, attn in enumerate(is_attn):
        p = f"model.layers.{l}"
        if attn:
            put(f"{p}.self_attn.q_proj.weight", (c.q_dim, c.dim))
            put(f"{p}.self_attn.k_proj.weight", (c.kv_dim, c.dim))
            put(f"{p}.self_attn.v_proj.weight", (c.kv_dim, c.dim))
            put(f"{p}.self_attn.out_proj.weight", (c.dim, c.q_dim))
            put(f"{p}.self_attn.q_layernorm.weight", (c.head_dim,), 1.0)
            put(f"{p}.self_attn.k_layernorm.weight", (c.head_dim,), 1.0)
        else:
            put(f"{p}.conv.in_proj.weight", (3 * c.dim, c.dim))
            put(f"{p}.conv.out_proj.weight", (c.dim, c.dim))
            put(f"{p}.conv.conv.weight", conv_shape or (c.dim, 1, k), 0.2)
        put(f"{p}.operator_norm.weight", (c.dim,), 1.0)
        put(f"{p}.ffn_norm.weight", (c.dim,), 1.0)
        put(f"{p}.feed_forward.w1.weight", (c.hidden_dim, c.dim))
        put(f"{p}.feed_forward.w2.weight", (c.dim, c.hidden_dim))
        put(f"{p}.feed_forward.w3.weight", (c.hidden_dim, c.dim))
    return t
