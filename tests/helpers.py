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
