"""Independent pins of the model schedules the oracle restates
(src/arch/llm/llama.rs:786-862, src/arch/llm/lfm2.rs:380-477).

The oracle's cpu and reference backends share one driver, so their agreement
cannot catch a slip in that driver (a swapped norm, gate/up swapped, a
dropped residual), and the GPU, checked against the oracle, would reproduce
it. Two checks written apart from oracle.cpp's driver:

1. The forward steps written again here, line by line from the Rust, over the
   oracle backend's trait ops: it must equal the oracle model bit for bit.
2. A float64 numpy forward of the same f32 weights, no oracle code at all
   (RMSNorm, per-head qk_norm, half-split RoPE, softmax attention, SwiGLU,
   LFM2's gated short convolution): it must track the oracle's reference
   backend within 1e-4 of the largest logit, while the same forward with a
   plausible schedule mistake lands far outside that.
"""

import numpy as np
import pytest

import oracle as O


def _close_rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))) /
                 max(1.0, float(np.max(np.abs(b)))))


# ---- 1. the Rust forward over the oracle backend's ops -----------------------

def _llama_step(b, c, w, bufs, token, pos):
    """llama.rs:786-862, one call = one token."""
    dim, hidden, qd, kvd, hs = c.dim, c.hidden_dim, c.q_dim, c.kv_dim, c.head_dim
    x, xb, q, k, v, attn, att, o, gate, up, mlp, logits = (bufs[n] for n in (
        "x", "xb", "q", "k", "v", "attn", "att", "o", "gate", "up", "mlp", "logits"))
    b.embed(token, x, 0)
    for l in range(c.n_layers):
        n = bufs["norms"][l]
        b.rms_norm(xb, x, n["att"], 1, dim, c.rms_eps)
        # project_qkv's default: three projects of the same x (mod.rs:326-330)
        b.project(l, "q", xb, q, 1)
        b.project(l, "k", xb, k, 1)
        b.project(l, "v", xb, v, 1)
        if "q" in n:
            b.qk_norm(q, 1, qd, hs, n["q"], c.rms_eps)
        if "k" in n:
            b.qk_norm(k, 1, kvd, hs, n["k"], c.rms_eps)
        b.rope(q, k, qd, kvd, 1, [pos], hs, c.rope_theta, c.rope_interleaved)
        b.kv_write(l, [pos], k, v, 1)
        b.attention(q, attn, att, l, [(0, pos, 0, 0)], c.n_heads, c.kv_mul, hs, kvd, c.seq_len)
        b.project(l, "o", attn, o, 1)
        b.add_in_place(x, o, dim)
        b.rms_norm(xb, x, n["ffn"], 1, dim, c.rms_eps)
        b.project(l, "gate", xb, gate, 1)
        b.project(l, "up", xb, up, 1)
        b.silu_mul(gate, up, hidden)
        b.project(l, "down", gate, mlp, 1)
        b.add_in_place(x, mlp, dim)
    b.rms_norm(xb, x, bufs["final"], 1, dim, c.rms_eps)
    b.logits(xb, logits)
    return b.read(logits, c.vocab_size)


def _lfm2_step(b, c, w, bufs, token, pos):
    """lfm2.rs:380-477, one call = one token."""
    dim, hidden, qd, kvd, hs = c.dim, c.hidden_dim, c.q_dim, c.kv_dim, c.head_dim
    x, xb, q, k, v, attn, att, o, gate, up, mlp, logits = (bufs[n] for n in (
        "x", "xb", "q", "k", "v", "attn", "att", "o", "gate", "up", "mlp", "logits"))
    bcx, h, co, cy = bufs["bcx"], bufs["h"], bufs["co"], bufs["cy"]
    b.embed(token, x, 0)
    for l in range(c.n_layers):
        n = bufs["norms"][l]
        b.rms_norm(xb, x, n["att"], 1, dim, c.rms_eps)
        if w.is_attention[l]:
            b.project(l, "q", xb, q, 1)
            b.project(l, "k", xb, k, 1)
            b.project(l, "v", xb, v, 1)
            b.qk_norm(q, 1, qd, hs, n["q"], c.rms_eps)
            b.qk_norm(k, 1, kvd, hs, n["k"], c.rms_eps)
            b.rope(q, k, qd, kvd, 1, [pos], hs, c.rope_theta, c.rope_interleaved)
            b.kv_write(l, [pos], k, v, 1)
            b.attention(q, attn, att, l, [(0, pos, 0, 0)], c.n_heads, c.kv_mul, hs, kvd, c.seq_len)
            b.project(l, "o", attn, o, 1)
            b.add_in_place(x, o, dim)
        else:
            b.project(l, "conv_in", xb, bcx, 1)
            b.mul(h, 0, bcx, 0, bcx, 2 * dim, dim)  # B * x: first and last thirds
            kw = w.layers[l]["conv_kernel"]
            b.conv_decode(co, h, n["conv"], n["ring"], dim, kw.shape[1])
            b.mul(cy, 0, bcx, dim, co, 0, dim)  # C * conv: the middle third
            b.project(l, "conv_out", cy, o, 1)
            b.add_in_place(x, o, dim)
        b.rms_norm(xb, x, n["ffn"], 1, dim, c.rms_eps)
        b.project(l, "gate", xb, gate, 1)
        b.project(l, "up", xb, up, 1)
        b.silu_mul(gate, up, hidden)
        b.project(l, "down", gate, mlp, 1)
        b.add_in_place(x, mlp, dim)
    b.rms_norm(xb, x, bufs["final"], 1, dim, c.rms_eps)
    b.logits(xb, logits)
    return b.read(logits, c.vocab_size)


def _buffers(b, c, w):
    bufs = {name: b.alloc(n) for name, n in [
        ("x", c.dim), ("xb", c.dim), ("q", c.q_dim), ("k", c.kv_dim), ("v", c.kv_dim), ("attn", c.q_dim),
        ("att", c.n_heads * c.seq_len), ("o", c.dim), ("gate", c.hidden_dim), ("up", c.hidden_dim),
        ("mlp", c.dim), ("logits", c.vocab_size), ("bcx", 3 * c.dim), ("h", c.dim), ("co", c.dim),
        ("cy", c.dim)]}
    norms = []
    for l in range(c.n_layers):
        d = w.layers[l]
        n = {"att": b.upload(d["norm_att"]), "ffn": b.upload(d["norm_ffn"])}
        for which in ("q", "k"):
            if "norm_" + which in d:
                n[which] = b.upload(d["norm_" + which])
        if "conv_kernel" in d:
            kw = d["conv_kernel"]
            n["conv"] = b.upload(kw)
            n["ring"] = b.upload(np.zeros((kw.shape[1] - 1) * c.dim, np.float32))  # seeded zero (lfm2.rs:315-321)
        norms.append(n)
    bufs["norms"] = norms
    bufs["final"] = b.upload(w.final_norm)
    return bufs


TOKENS = [3, 17, 0, 29, 8, 8, 21, 5, 30, 12]


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_llama_forward_restated_from_rust_matches_the_oracle(storage):
    c = O.backends_config()
    w = O.backends_weights(c, storage)  # distinct att/ffn/final norms, qk_norm, untied classifier
    model = O.Model(c, w, "cpu")
    b = O.Backend("cpu", w, n_layers=c.n_layers, kv_dim=c.kv_dim, seq_len=c.seq_len)
    bufs = _buffers(b, c, w)
    for pos, tok in enumerate(TOKENS):
        got = _llama_step(b, c, w, bufs, tok, pos)
        want = model.forward(tok, pos)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"position {pos}"


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_lfm2_forward_restated_from_rust_matches_the_oracle(storage):
    c = O.lfm2_config()
    w = O.lfm2_weights(c, [False, True], storage)  # a conv layer, then an attention layer
    model = O.Model(c, w, "cpu", lfm2=True)
    b = O.Backend("cpu", w, n_layers=c.n_layers, kv_dim=c.kv_dim, seq_len=c.seq_len)
    bufs = _buffers(b, c, w)
    for pos, tok in enumerate(TOKENS):
        got = _lfm2_step(b, c, w, bufs, tok, pos)
        want = model.forward(tok, pos)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"position {pos}"


# ---- 2. a float64 forward with no oracle code ---------------------------------

def _rms(x, wt, eps):
    return wt * (x / np.sqrt(np.mean(x * x) + eps))


def _rope_half(v, pos, hs, theta):
    v = v.reshape(-1, hs).copy()
    half = hs // 2
    ang = pos * theta ** (-2.0 * np.arange(half) / hs)
    lo, hi = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = lo * np.cos(ang) - hi * np.sin(ang)
    v[:, half:] = lo * np.sin(ang) + hi * np.cos(ang)
    return v.ravel()


def _attend(q, keys, vals, n_heads, kv_mul, hs):
    out = np.empty(n_heads * hs)
    for h in range(n_heads):
        kh = keys[:, (h // kv_mul) * hs:(h // kv_mul + 1) * hs]
        vh = vals[:, (h // kv_mul) * hs:(h // kv_mul + 1) * hs]
        s = kh @ q[h * hs:(h + 1) * hs] / np.sqrt(hs)
        p = np.exp(s - s.max())
        out[h * hs:(h + 1) * hs] = (p / p.sum()) @ vh
    return out


def _f64_forward(c, w, tokens, lfm2=False, mistake=None):
    """Logits at every position. `mistake` plants one schedule slip here, in
    this float64 model, to show the 1e-4 check tells it apart."""
    f = lambda m: np.asarray(m.to_f32(), np.float64)
    emb = f(w.embedding)
    cls = f(w.classifier) if w.classifier is not None else emb
    L, hs = c.n_layers, c.head_dim
    P = [{k: (f(v) if isinstance(v, O.Matrix) else np.asarray(v, np.float64)) for k, v in d.items()}
         for d in w.layers]
    keys = [np.zeros((c.seq_len, c.kv_dim)) for _ in range(L)]
    vals = [np.zeros((c.seq_len, c.kv_dim)) for _ in range(L)]
    hist = [np.zeros((0, c.dim)) for _ in range(L)]
    out = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        for l in range(L):
            p = P[l]
            n_att, n_ffn = (p["norm_ffn"], p["norm_att"]) if mistake == "swap_norms" else (p["norm_att"], p["norm_ffn"])
            xb = _rms(x, n_att, c.rms_eps)
            if not lfm2 or w.is_attention[l]:
                q, k, v = p["q"] @ xb, p["k"] @ xb, p["v"] @ xb
                if "norm_q" in p:
                    q = np.concatenate([_rms(q[i:i + hs], p["norm_q"], c.rms_eps) for i in range(0, len(q), hs)])
                    k = np.concatenate([_rms(k[i:i + hs], p["norm_k"], c.rms_eps) for i in range(0, len(k), hs)])
                q, k = _rope_half(q, pos, hs, c.rope_theta), _rope_half(k, pos, hs, c.rope_theta)
                keys[l][pos], vals[l][pos] = k, v
                a = _attend(q, keys[l][:pos + 1], vals[l][:pos + 1], c.n_heads, c.kv_mul, hs)
                y = p["o"] @ a
            else:
                bcx = p["conv_in"] @ xb
                B, Cg, xx = bcx[:c.dim], bcx[c.dim:2 * c.dim], bcx[2 * c.dim:]
                kw = p["conv_kernel"]  # [dim, k]: tap j meets the input k - 1 - j rows back
                hist[l] = np.vstack([hist[l], B * xx])
                kk = kw.shape[1]
                conv = np.zeros(c.dim)
                for j in range(kk):
                    t = len(hist[l]) - kk + j
                    if t >= 0:
                        conv += kw[:, j] * hist[l][t]
                y = p["conv_out"] @ (Cg * conv)
            if mistake != "drop_residual" or l != L - 1:
                x = x + y
            else:
                x = y
            xb = _rms(x, n_ffn, c.rms_eps)
            g, u = p["gate"] @ xb, p["up"] @ xb
            if mistake == "swap_gate_up":
                g, u = u, g
            x = x + p["down"] @ (g / (1.0 + np.exp(-g)) * u)
        out.append(cls @ _rms(x, w.final_norm, c.rms_eps))
    return out


@pytest.mark.parametrize("arch", ["llama", "lfm2"])
def test_float64_forward_tracks_the_oracle_reference_backend(arch):
    if arch == "llama":
        c = O.backends_config()
        c.n_layers = 1
        w = O.backends_weights(c, "f32")
        model = O.Model(c, w, "reference")
    else:
        c = O.lfm2_config()
        w = O.lfm2_weights(c, [False, True], "f32")
        model = O.Model(c, w, "reference", lfm2=True)
    want = [model.forward(tok, pos).copy() for pos, tok in enumerate(TOKENS)]
    got = _f64_forward(c, w, TOKENS, lfm2=arch == "lfm2")
    for pos in range(len(TOKENS)):
        assert _close_rel(got[pos], want[pos]) <= 1e-4, f"position {pos}: {_close_rel(got[pos], want[pos])}"
    # each planted slip moves the logits far past the tolerance somewhere
    for mistake in ("swap_norms", "swap_gate_up", "drop_residual"):
        bad = _f64_forward(c, w, TOKENS, lfm2=arch == "lfm2", mistake=mistake)
        worst = max(_close_rel(bad[p], want[p]) for p in range(len(TOKENS)))
        assert worst > 1e-2, f"{mistake} not told apart ({worst})"
