"""Bit-exact parity at the widths of BASELINE.json's configs that the smaller
model tests do not reach: the LFM2-700M (cfg4) and Qwen3-0.6B (cfg5)
projection shapes at 1, 64 and 2048 rows, their classifiers, the
2-layer LFM2 at 700M widths with an 8192-position context, the head_dim-128
batched decode, and the SmolLM2-360M (cfg2) model at full depth and
vocabulary with its cache filled to 512 positions.

Where a full-size oracle run would take minutes, the GPU computes the whole
shape and the oracle recomputes a seeded sample of (row, output) pairs from
the same bytes: every output is a function of its own row and weight row
only, so a sample is an exact check of the values it covers.
"""

import numpy as np
import pytest

import kernrt_amd as K
import oracle as O
from helpers import assert_bits_equal, gaussian_weights, gpu_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    h = K.open("hip")
    yield h
    h.close()


def random_q8(storage, n, k, seed):
    """Random Q8 bytes (any int8 in [-127, 127] and positive scales are valid
    Q8_0 data; Q8_0x4 records carry f16 scale bits). Returns the product-side
    matrix and a function that builds the oracle matrix of a row subset."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    if storage == "q8_0":
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        s = rng.uniform(1e-4, 3e-4, size=(n, nb)).astype(np.float32)
        prod = K.Q8Matrix("q8_0", n, k, quants=q.ravel(), scales=s.ravel())

        def sub(rows):
            return O.Matrix.from_q8_0(q[rows].ravel(), s[rows].ravel(), len(rows), k)
        return prod, sub
    rec = np.empty((n // 4, nb, 136), np.uint8)
    sc = rng.uniform(1e-4, 3e-4, size=(n // 4, nb, 4)).astype(np.float16)
    rec[:, :, :8] = sc.view(np.uint8).reshape(n // 4, nb, 8)
    rec[:, :, 8:] = rng.integers(-127, 128, size=(n // 4, nb, 128), dtype=np.int8).view(np.uint8)
    prod = K.Q8Matrix("q8_0x4", n, k, blocks=rec.ravel())

    def sub(groups):
        return O.Matrix.from_q8_0x4_blocks(rec[groups].ravel(), 4 * len(groups), k)
    return prod, sub


def sampled_check(storage, n, k, sub, x, got, seed, what, n_rows=12, n_out=192, logits=False):
    rng = np.random.default_rng(seed)
    m = x.shape[0]
    ridx = np.sort(rng.choice(m, size=min(m, n_rows), replace=False))
    if storage == "q8_0":
        oidx = np.sort(rng.choice(n, size=min(n, n_out), replace=False))
        om = sub(oidx)
    else:
        groups = np.sort(rng.choice(n // 4, size=min(n // 4, n_out // 4), replace=False))
        oidx = (groups[:, None] * 4 + np.arange(4)[None, :]).ravel()
        om = sub(groups)
    if logits:
        assert m == 1
        want = om.logits_cpu(x[0])[None, :]
    else:
        want = om.project_cpu(x[ridx])
    assert_bits_equal(got[ridx][:, oidx] if not logits else got[:, oidx], want, what)


# (out_dim, in_dim): cfg5 q / k,v / gate,up / o / down, cfg4 conv-in,gate,up / out,o / k,v / down
SHAPES = [(2048, 1024), (1024, 1024), (3072, 1024), (1024, 2048), (1024, 3072),
          (4608, 1536), (1536, 1536), (512, 1536), (1536, 4608)]


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("rows", [1, 64, 2048])
def test_project_at_cfg4_cfg5_shapes(hip, storage, shape, rows):
    n, k = shape
    seed = n * 7 + k * 3 + rows
    prod, sub = random_q8(storage, n, k, seed)
    mat = hip.upload_matrix(prod)
    x = np.random.default_rng(seed + 1).normal(size=(rows, k)).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero activation block
    y = hip.alloc(rows * n)
    hip.matmul(mat, hip.upload(x), y, rows)
    got = hip.read(y, rows * n).reshape(rows, n)
    sampled_check(storage, n, k, sub, x, got, seed + 2, f"{storage} {n}x{k} rows={rows}")
    hip.free_matrix(mat)


@pytest.mark.parametrize("storage,n,k,rows", [("q8_0x4", 65536, 1536, 1), ("q8_0", 151936, 1024, 1),
                                              ("q8_0", 151936, 1024, 64)])
def test_classifiers_at_cfg4_cfg5_vocab(hip, storage, n, k, rows):
    # cfg4's tied 65536-row Q8_0x4 classifier through logits (x86 semantics,
    # quant.rs:223-236) and cfg5's 151936-row Q8_0 lm_head, one row and the
    # 64-row batched-decode GEMM
    seed = n + rows
    prod, sub = random_q8(storage, n, k, seed)
    mat = hip.upload_matrix(prod)
    x = np.random.default_rng(seed + 1).normal(size=(rows, k)).astype(np.float32)
    y = hip.alloc(rows * n)
    if rows == 1:
        hip.classify(mat, hip.upload(x[0]), y)
    else:
        hip.matmul(mat, hip.upload(x), y, rows)
    got = hip.read(y, rows * n).reshape(rows, n)
    sampled_check(storage, n, k, sub, x, got, seed + 2, f"classifier {n}x{k} rows={rows}", n_out=1024,
                  logits=rows == 1)
    hip.free_matrix(mat)


def fill_cache(models, c, layers, n_pos, seed):
    """The same N(0, 1) keys and values into cache positions [0, n_pos) of
    `layers` on every model (GPU `K.Model` or oracle `O.Model`)."""
    rng = np.random.default_rng(seed)
    kv = c.n_kv_heads * c.head_dim
    for l in layers:
        keys = rng.normal(size=n_pos * kv).astype(np.float32)
        vals = rng.normal(size=n_pos * kv).astype(np.float32)
        for mdl in models:
            up = mdl.backend.kv_upload if isinstance(mdl, K.Model) else mdl.kv_upload
            up(0, l * c.seq_len * kv, keys)
            up(1, l * c.seq_len * kv, vals)


LFM2_700M = dict(dim=1536, hidden_dim=4608, n_layers=2, n_heads=24, n_kv_heads=8, vocab_size=4096, seq_len=8192,
                 rms_eps=1e-5, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=64)


@pytest.mark.parametrize("storage", ["q8_0x4", "q8_0"])
def test_lfm2_700m_widths_long_context(storage):
    # cfg4's widths (dim 1536, 24/8 heads, hidden 4608, QK-norm, context
    # 8192) with one conv and one attention layer: the fused decode at dim
    # 1536 (two values per thread in the projection producer, the conv block),
    # a chunked prefill at position 5000 (the conv history from the ring for
    # Q8_0, zero-padded for Q8_0x4, as the reference does), and decode over
    # 5000+ cached positions with an 8192-position context, where decode
    # attention runs as one launch with a device window
    c = O.Config(**LFM2_700M)
    ow = gaussian_weights(c, storage, seed=70, lfm2_mask=[False, True], qk_norm=True, norms="uniform")
    gpu, cpu = gpu_model(c, ow, lfm2=True), O.Model(c, ow, "cpu", lfm2=True)
    start = 5000
    fill_cache([gpu, cpu], c, [1], start, seed=71)
    prompt = [int(t) for t in np.random.default_rng(72).integers(0, c.vocab_size, size=7)]
    assert_bits_equal(gpu.prefill(prompt[:3], start), cpu.prefill(prompt[:3], start), "prefill chunk 1")
    assert_bits_equal(gpu.prefill(prompt[3:], start + 3), cpu.prefill(prompt[3:], start + 3), "prefill chunk 2")
    pos = start + len(prompt)
    tok = 11
    for i in range(4):
        a, b = gpu.forward(tok, pos + i), cpu.forward(tok, pos + i)
        assert_bits_equal(a, b, f"decode at {pos + i}")
        tok = O.argmax(b)
    # then a prefill after decoding: the ring carries the decoded rows
    p2 = [3, 9]
    assert_bits_equal(gpu.prefill(p2, pos + 4), cpu.prefill(p2, pos + 4), "prefill after decode")
    got = gpu.generate_greedy(tok, pos + 6, 6, use_graph=True)
    want = []
    for i in range(6):
        tok = O.argmax(cpu.forward(tok, pos + 6 + i))
        want.append(tok)
    assert list(got) == want


@pytest.mark.parametrize("mask", [[False, False], [False, True]])
def test_lfm2_q8_0_chunked_prefill_continues_the_ring(mask):
    # lfm2.rs:490-495: a Q8_0 LFM2 prefills token by token, so the conv ring
    # carries across prefill calls; a batched prefill must give the same bits
    c = O.lfm2_config()
    ow = O.lfm2_weights(c, mask, "q8_0")
    gpu, cpu = gpu_model(c, ow, lfm2=True), O.Model(c, ow, "cpu", lfm2=True)
    prompt = [5, 11, 2, 30, 7, 7, 19, 1, 24]
    assert_bits_equal(gpu.prefill(prompt[:4], 0), cpu.prefill(prompt[:4], 0), "chunk 1")
    assert_bits_equal(gpu.prefill(prompt[4:5], 4), cpu.prefill(prompt[4:5], 4), "one-token chunk")
    assert_bits_equal(gpu.prefill(prompt[5:], 5), cpu.prefill(prompt[5:], 5), "chunk 3")
    for i, t in enumerate([3, 8]):
        assert_bits_equal(gpu.forward(t, 9 + i), cpu.forward(t, 9 + i), f"decode {i}")


def test_lfm2_q8_0x4_chunked_prefill_follows_the_batched_reference():
    # lfm2.rs:587-603: a batched prefill zero-pads the conv history and
    # copies its last k - 1 rows into the ring's tail; a later chunk does the
    # same again (the reference's own behaviour for q8_0x4, reproduced)
    c = O.lfm2_config()
    ow = O.lfm2_weights(c, [False, True], "q8_0x4")
    gpu, cpu = gpu_model(c, ow, lfm2=True), O.Model(c, ow, "cpu", lfm2=True)
    prompt = [5, 11, 2, 30, 7, 7, 19, 1, 24]
    assert_bits_equal(gpu.prefill(prompt[:4], 0), cpu.prefill(prompt[:4], 0), "chunk 1")
    assert_bits_equal(gpu.prefill(prompt[4:5], 4), cpu.prefill(prompt[4:5], 4), "one-token chunk")
    assert_bits_equal(gpu.prefill(prompt[5:], 5), cpu.prefill(prompt[5:], 5), "chunk 3")
    assert_bits_equal(gpu.forward(3, 9), cpu.forward(3, 9), "decode")


QWEN3_SMALL = dict(dim=1024, hidden_dim=512, n_layers=1, n_heads=16, n_kv_heads=8, vocab_size=1024,
                   rms_eps=1e-6, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=128)


@pytest.mark.parametrize("n_seq", [4, 9])
def test_decode_batch_head_dim_128(n_seq):
    # cfg5's attention shape (16 query / 8 KV heads of 128, QK-norm) in the
    # batched decode: sequence s owns slots [s * room, (s + 1) * room), its
    # cache filled to a length of its own; each step's row s must equal
    # forward() of that sequence alone. 4 rows take the GEMV path, 9 the GEMM.
    room = 400
    c = O.Config(seq_len=room * n_seq, **QWEN3_SMALL)
    ow = gaussian_weights(c, "q8_0", seed=80 + n_seq, qk_norm=True, norms="uniform")
    rng = np.random.default_rng(n_seq)
    ctx = [int(n) for n in rng.integers(200, room - 8, size=n_seq)]
    g = gpu_model(c, ow)
    cpus = [O.Model(c, ow, "cpu") for _ in range(n_seq)]
    kv = c.n_kv_heads * c.head_dim
    for s in range(n_seq):
        keys = rng.normal(size=ctx[s] * kv).astype(np.float32)
        vals = rng.normal(size=ctx[s] * kv).astype(np.float32)
        g.backend.kv_upload(0, s * room * kv, keys)
        g.backend.kv_upload(1, s * room * kv, vals)
        cpus[s].kv_upload(0, 0, keys)
        cpus[s].kv_upload(1, 0, vals)
    for t in range(4):
        toks = [int(v) for v in rng.integers(0, c.vocab_size, size=n_seq)]
        got = g.decode_batch(toks, [ctx[s] + t for s in range(n_seq)], [s * room + ctx[s] + t for s in range(n_seq)],
                             [s * room for s in range(n_seq)])
        for s in range(n_seq):
            assert_bits_equal(got[s], cpus[s].forward(toks[s], ctx[s] + t), f"step {t} sequence {s}")


def test_decode_batch_windows_past_2048():
    # the batched decode's split attention with windows of 2100-2600
    # positions (past the 2048 of its first form; the LDS holds the score rows
    # and one V tile): each step's rows must equal forward() of each sequence
    room = 2700
    n_seq = 3
    c = O.Config(seq_len=room * n_seq, **QWEN3_SMALL)
    ow = gaussian_weights(c, "q8_0", seed=91, qk_norm=True, norms="uniform")
    rng = np.random.default_rng(92)
    ctx = [2100, 2400, 2650]
    g = gpu_model(c, ow)
    cpus = [O.Model(c, ow, "cpu") for _ in range(n_seq)]
    kv = c.n_kv_heads * c.head_dim
    for s in range(n_seq):
        keys = rng.normal(size=ctx[s] * kv).astype(np.float32)
        vals = rng.normal(size=ctx[s] * kv).astype(np.float32)
        g.backend.kv_upload(0, s * room * kv, keys)
        g.backend.kv_upload(1, s * room * kv, vals)
        cpus[s].kv_upload(0, 0, keys)
        cpus[s].kv_upload(1, 0, vals)
    for t in range(2):
        toks = [int(v) for v in rng.integers(0, c.vocab_size, size=n_seq)]
        got = g.decode_batch(toks, [ctx[s] + t for s in range(n_seq)], [s * room + ctx[s] + t for s in range(n_seq)],
                             [s * room for s in range(n_seq)])
        for s in range(n_seq):
            assert_bits_equal(got[s], cpus[s].forward(toks[s], ctx[s] + t), f"step {t} sequence {s}")


SMOLLM2_360M = dict(dim=960, hidden_dim=2560, n_layers=32, n_heads=15, n_kv_heads=5, vocab_size=49152, seq_len=1024,
                    rms_eps=1e-5, rope_theta=100_000.0, rope_interleaved=False, head_dim=64)


def test_cfg2_full_depth_and_vocabulary():
    # the benchmark's model at full size: 32 layers, 49152-token tied
    # classifier, Q8_0x4, cache filled to 512 positions; forward() and the
    # captured greedy step graph must match the oracle token for token
    c = O.Config(**SMOLLM2_360M)
    ow = gaussian_weights(c, "q8_0x4", seed=360)
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    fill_cache([gpu, cpu], c, range(c.n_layers), 512, seed=361)
    tok = 1234
    for i in range(3):
        a, b = gpu.forward(tok, 512 + i), cpu.forward(tok, 512 + i)
        assert_bits_equal(a, b, f"decode at {512 + i}")
        tok = O.argmax(b)
    got = gpu.generate_greedy(tok, 515, 4, use_graph=True)
    want = []
    for i in range(4):
        tok = O.argmax(cpu.forward(tok, 515 + i))
        want.append(tok)
    assert list(got) == want
