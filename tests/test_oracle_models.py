"""The reference's cross-backend invariants (tests/backends.rs, lfm2.rs tests,
llama.rs tests) run on the oracle's Cpu and Reference restatements (CPU only).

Cpu and Reference share no projection or attention arithmetic (int8 vs f32,
four-chain FMA dot vs plain loop), so their agreement pins the restated
drivers and non-hot ops the same way it pins the reference's.
"""

import numpy as np

import oracle as O

PROMPT = [5, 11, 2, 30, 7, 7, 19, 1, 24]


def max_diff(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))))


def model(backend, storage="f32"):
    c = O.backends_config()
    return O.Model(c, O.backends_weights(c, storage), backend)


def test_backends_agree_on_decode():
    # tests/backends.rs:128-148
    cpu, ref = model("cpu"), model("reference")
    for pos, tok in enumerate([3, 17, 0, 29, 8, 8, 21]):
        a, b = cpu.forward(tok, pos), ref.forward(tok, pos)
        assert max_diff(a, b) <= 1e-3
        assert O.argmax(a) == O.argmax(b)


def test_backends_agree_on_batched_prefill():
    # tests/backends.rs:153-174
    for name in ["cpu", "reference"]:
        got = model(name).prefill(PROMPT, 0)
        seq = model(name)
        for pos, tok in enumerate(PROMPT):
            want = seq.forward(tok, pos)
        assert max_diff(got, want) <= 1e-3
        assert O.argmax(got) == O.argmax(want)


def test_backends_agree_on_shared_prefix():
    # tests/backends.rs:179-192
    prefix = [4, 9, 14]
    suffixes = [[20, 6], [12, 12, 12, 12], [31]]
    a = model("cpu").prefill_shared(prefix, suffixes)
    b = model("reference").prefill_shared(prefix, suffixes)
    assert a.shape == b.shape
    for i in range(len(suffixes)):
        assert max_diff(a[i], b[i]) <= 1e-3, f"leaf {i}"


def test_shared_prefix_matches_spelled_out_leaves():
    # llama.rs:596-599: prefill_shared equals prefill_multi over concatenated leaves
    prefix = [4, 9, 14]
    suffixes = [[20, 6], [12, 12, 12, 12], [31]]
    for storage in ["f32", "q8_0x4"]:
        shared = model("cpu", storage).prefill_shared(prefix, suffixes)
        multi = model("cpu", storage).prefill_multi([prefix + s for s in suffixes])
        assert max_diff(shared, multi) <= 1e-5


def test_cpu_prefill_matches_decode_when_exactness_is_promised():
    # tests/backends.rs:234-274 (the f32-copy cases are not restated)
    for storage in ["f32", "q8_0", "q8_0x4"]:
        got = model("cpu", storage).prefill(PROMPT, 0)
        seq = model("cpu", storage)
        for pos, tok in enumerate(PROMPT):
            want = seq.forward(tok, pos)
        assert max_diff(got, want) <= 1e-3, storage
        assert O.argmax(got) == O.argmax(want), storage


def test_q8_paths_track_the_reference_backend():
    # tests/backends.rs:390-426 standard (5e-2 + argmax) for the int8 paths
    for storage in ["q8_0", "q8_0x4"]:
        cpu, ref = model("cpu", storage), model("reference", storage)
        for pos, tok in enumerate(PROMPT):
            a, b = cpu.forward(tok, pos), ref.forward(tok, pos)
            assert max_diff(a, b) <= 5e-2, (storage, pos)
            assert O.argmax(a) == O.argmax(b), (storage, pos)


def test_q8x4_batched_prefill_is_bit_identical_to_decode():
    # quant.rs:238-244: the batched kernel keeps the decode order per output
    got = model("cpu", "q8_0x4").prefill(PROMPT, 0)
    seq = model("cpu", "q8_0x4")
    for pos, tok in enumerate(PROMPT):
        want = seq.forward(tok, pos)
    assert np.array_equal(got, want)


def test_lfm2_prefill_matches_decode_per_layer_kind():
    # lfm2.rs:794-824, plus the Q8 storages
    prompt = [5, 11, 2, 30]
    for storage in ["f32", "q8_0x4"]:
        for mask in ([True, True], [False, False], [False, True]):
            c = O.lfm2_config()
            got = O.Model(c, O.lfm2_weights(c, mask, storage), "cpu", lfm2=True).prefill(prompt, 0)
            seq = O.Model(c, O.lfm2_weights(c, mask, storage), "cpu", lfm2=True)
            for pos, tok in enumerate(prompt):
                want = seq.forward(tok, pos)
            assert max_diff(got, want) <= 1e-3, (storage, mask)


def test_lfm2_cpu_agrees_with_reference():
    # lfm2.rs:871-940 standard, run on the oracle's two backends
    prompt = [5, 11, 2, 30, 7, 7, 19, 1, 24]
    c = O.lfm2_config()
    mask = [False, True]
    cpu = O.Model(c, O.lfm2_weights(c, mask), "cpu", lfm2=True)
    ref = O.Model(c, O.lfm2_weights(c, mask), "reference", lfm2=True)
    for pos, tok in enumerate(prompt):
        a, b = cpu.forward(tok, pos), ref.forward(tok, pos)
        assert max_diff(a, b) <= 1e-3
        assert O.argmax(a) == O.argmax(b)


def test_conv_prefill_matches_stepped_decode():
    # lfm2.rs:830-865
    b = O.Backend("cpu")
    dim, k, rows = 8, 3, 5
    h = np.sin(np.arange(rows * dim, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    kw = np.cos(np.arange(dim * k, dtype=np.float32) * np.float32(0.11)).astype(np.float32)
    hb, kb = b.upload(h), b.upload(kw)
    out = b.alloc(rows * dim)
    b.conv_prefill(out, hb, kb, rows, dim, k)
    got = b.read(out, rows * dim)
    state = b.alloc(dim * (k - 1))
    want = np.zeros(rows * dim, np.float32)
    for r in range(rows):
        xr = b.upload(h[r * dim:(r + 1) * dim])
        orow = b.alloc(dim)
        b.conv_decode(orow, xr, kb, state, dim, k)
        want[r * dim:(r + 1) * dim] = b.read(orow, dim)
    assert max_diff(got, want) <= 1e-5


def test_qk_norm_normalizes_each_head_separately():
    # llama.rs:954-977
    b = O.Backend("cpu")
    data = np.array([3.0, 0.0, 0.0, 0.0, 0.1, 0.1, 0.1, 0.1], np.float32)
    v, w = b.upload(data), b.upload(np.ones(4, np.float32))
    b.qk_norm(v, 1, 8, 4, w, 0.0)
    out = b.read(v, 8)
    rms = lambda h: np.sqrt(np.mean(h * h))
    assert abs(rms(out[:4]) - 1) < 1e-5 and abs(rms(out[4:]) - 1) < 1e-5
    assert abs(out[0] - 2.0) < 1e-5 and np.all(out[1:4] == 0)


def test_rope_styles_preserve_norms():
    # llama.rs:981-1015
    q = np.array([0.3, -0.7, 1.1, 0.2, -0.4, 0.9, 0.5, -0.1], np.float32)
    for interleaved in [True, False]:
        b = O.Backend("cpu")
        qb, kb = b.upload(q), b.upload(np.zeros(8, np.float32))
        b.rope(qb, kb, 8, 8, 1, [3], 4, 10_000.0, interleaved)
        out = b.read(qb, 8)
        assert abs(np.sum(out * out) - np.sum(q * q)) < 1e-5
