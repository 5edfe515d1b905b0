"""The acceptance check of the decode path at its full configured size
the SmolLM2-360M-shaped model -- 32 layers, dim 960,
15 / 5 heads, hidden 2560, vocab 49152, Q8_0x4 weights N(0, 0.02), the KV
cache pre-filled to 512 positions from N(0, 1) -- decodes 256 greedy tokens
through the captured step graph, and the oracle's cpu backend, given the very
weight bytes and cache read back from the device, decodes the same 256
tokens (greedy = argmax with ties to the last maximal index,
src/generate.rs:70-77; the model step src/arch/llm/llama.rs:786-862).

About two minutes on one host core for the oracle's 256 steps."""

import numpy as np
import pytest

import bench
import kernrt_amd as K
import oracle as O

pytestmark = pytest.mark.gpu

STEPS = 256


@pytest.mark.timeout(900)
def test_cfg2_full_size_256_greedy_tokens_match_the_oracle():
    hip, model, c = bench.synthetic_model(K, bench.CFG2, "q8_0x4", seed=2)
    hip.kv_synthetic(bench.PREFILL_POS, seed=5)
    token0 = int(np.random.default_rng(2).integers(0, c.vocab_size))
    gpu_tokens = [int(t) for t in model.generate_greedy(token0, bench.PREFILL_POS, STEPS, use_graph=True)]
    # logits of the first step through forward() (the cache already holds
    # these positions: the same values are written again)
    gpu_logits0 = model.forward(token0, bench.PREFILL_POS).copy()

    # the same bytes into the oracle
    emb, handles = model.weight_handles
    w = O.Weights(c.n_layers)

    def omat(h):
        st, n, k = hip.matrix_shape(h)
        q, sc = hip.read_matrix(h)
        return O.Matrix.from_q8_0x4_blocks(K.backends.q8_0x4_records(q, sc), n, k)

    for l in range(c.n_layers):
        for name, h in handles[l].items():
            w.set_proj(l, name, omat(h))
        w.set_norm(l, "att", np.ones(c.dim, np.float32))
        w.set_norm(l, "ffn", np.ones(c.dim, np.float32))
    w.set_embedding(omat(emb))
    w.set_final_norm(np.ones(c.dim, np.float32))
    w.set_classifier(None)
    cpu = O.Model(O.Config(**bench.CFG2), w, "cpu")
    per = bench.PREFILL_POS * c.kv_dim
    for l in range(c.n_layers):
        for which in (0, 1):
            off = l * c.seq_len * c.kv_dim
            cpu.kv_upload(which, off, hip.kv_read(which, off, per))
    model.close()
    hip.close()

    tok = token0
    for i in range(STEPS):
        logits = cpu.forward(tok, bench.PREFILL_POS + i)
        if i == 0:
            assert np.array_equal(logits.view(np.uint32), gpu_logits0.view(np.uint32)), "step 0 logits"
        tok = O.argmax(logits)
        assert tok == gpu_tokens[i], f"greedy token {i} (position {bench.PREFILL_POS + i + 1})"
