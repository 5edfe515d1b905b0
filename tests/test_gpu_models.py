"""Model-level parity of the HIP backend through the C++ drivers, against the
oracle's Cpu backend driven by the oracle's restatement of the reference
drivers. Logits and hidden rows are compared as raw bits; greedy tokens must
be identical.

The reference's own cross-backend template (tests/backends.rs:331-481) asks a
GPU backend for 1e-3 against the scalar oracle plus identical argmax; the
int8 path here is held to bit equality with the cpu backend instead."""

import numpy as np
import pytest

import kernrt_amd as K
import oracle as O
from helpers import assert_bits_equal, gaussian_weights, gpu_model

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["fused", "unfused"])
def driver_mode(request, monkeypatch):
    """Every model test runs through both driver schedules: the fused kernels
    and the reference's op-by-op sequence of backend calls."""
    if request.param == "unfused":
        monkeypatch.setenv("KERNRT_HIP_UNFUSED", "1")
    else:
        monkeypatch.delenv("KERNRT_HIP_UNFUSED", raising=False)
    return request.param

PROMPT = [5, 11, 2, 30, 7, 7, 19, 1, 24]


def test_open_reports_the_hip_backend():
    hip = K.open("hip")
    assert hip.name() == "hip"
    assert hip.storage() == "f32"  # before prepare, like cpu.rs:101
    assert hip.device_name()
    hip.close()


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_decode_matches_the_cpu_backend_bitwise(storage):
    c = O.backends_config()
    ow = O.backends_weights(c, storage)
    gpu = gpu_model(c, ow)
    cpu = O.Model(c, ow, "cpu")
    ref = O.Model(c, ow, "reference")
    assert gpu.storage() == storage
    for pos, tok in enumerate([3, 17, 0, 29, 8, 8, 21]):
        assert_bits_equal(gpu.forward(tok, pos), cpu.forward(tok, pos), f"{storage} pos {pos}")
    # tests/backends.rs:390-426: the quantized GPU path against the scalar
    # oracle, 5e-2 and the same argmax, on that test's prompt
    gpu, ref = gpu_model(c, ow), O.Model(c, ow, "reference")
    for pos, tok in enumerate(PROMPT):
        a, r = gpu.forward(tok, pos), ref.forward(tok, pos)
        assert np.max(np.abs(a - r)) <= 5e-2 and O.argmax(a) == O.argmax(r), f"{storage} pos {pos}"


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_prefill_matches_stepped_decode_bitwise(storage):
    c = O.backends_config()
    ow = O.backends_weights(c, storage)
    got = gpu_model(c, ow).prefill(PROMPT, 0)
    want = O.Model(c, ow, "cpu").prefill(PROMPT, 0)
    assert_bits_equal(got, want, f"{storage} prefill vs oracle")
    stepped = gpu_model(c, ow)
    for pos, tok in enumerate(PROMPT):
        last = stepped.forward(tok, pos)
    assert_bits_equal(got, last, f"{storage} batched prefill vs decode loop")


def test_chunked_prefill_resumes_from_the_cache():
    # tests/end_to_end.rs:139- : a prompt in two chunks equals one pass
    c = O.backends_config()
    ow = O.backends_weights(c, "q8_0x4")
    one = gpu_model(c, ow).prefill(PROMPT, 0)
    m = gpu_model(c, ow)
    m.prefill(PROMPT[:4], 0)
    two = m.prefill(PROMPT[4:], 4)
    assert_bits_equal(two, one, "chunked prefill")


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_shared_prefix_and_multi_sequence(storage):
    # tests/backends.rs:179-192 and llama.rs:552-647
    c = O.backends_config()
    ow = O.backends_weights(c, storage)
    prefix, suffixes = [4, 9, 14], [[20, 6], [12, 12, 12, 12], [], [31]]
    assert_bits_equal(gpu_model(c, ow).prefill_shared(prefix, suffixes),
                      O.Model(c, ow, "cpu").prefill_shared(prefix, suffixes), "prefill_shared")
    seqs = [prefix + s for s in suffixes]
    assert_bits_equal(gpu_model(c, ow).prefill_multi(seqs), O.Model(c, ow, "cpu").prefill_multi(seqs),
                      "prefill_multi")


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("n_seq", [3, 9])
def test_decode_batch_matches_per_sequence_forward(storage, n_seq):
    # the batched decode step (krl_decode_batch): sequence s owns cache slots
    # [s * room, (s + 1) * room) and is decoded token by token, every step a
    # batch over the sequences still running; each row's logits must equal
    # forward() of that sequence run alone. Batches of 3 or fewer rows take
    # the GEMV path, 8 or more the int8 MFMA GEMM path.
    c = O.backends_config()
    ow = O.backends_weights(c, storage)
    rng = np.random.default_rng(n_seq)
    room = c.seq_len // n_seq
    seqs = [[int(t) for t in rng.integers(0, c.vocab_size, size=int(n))]
            for n in rng.integers(2, min(room, 7), size=n_seq)]
    g = gpu_model(c, ow)
    cpus = [O.Model(c, ow, "cpu") for _ in seqs]
    for t in range(max(len(s) for s in seqs)):
        live = [i for i, s in enumerate(seqs) if t < len(s)]
        got = g.decode_batch([seqs[i][t] for i in live], [t] * len(live), [i * room + t for i in live],
                             [i * room for i in live])
        for r, i in enumerate(live):
            assert_bits_equal(got[r], cpus[i].forward(seqs[i][t], t), f"decode_batch step {t} sequence {i}")


@pytest.mark.parametrize("n_seq", [3, 9])
def test_decode_batch_split_attention(n_seq):
    # batched decode with head_dim 64: rows whose windows belong to different
    # sequences take the two-launch split attention over many rows
    c = O.Config(dim=128, hidden_dim=128, n_layers=1, n_heads=2, n_kv_heads=1, vocab_size=64, seq_len=96 * n_seq,
                 rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0", seed=n_seq + 5)
    rng = np.random.default_rng(n_seq + 1)
    room = c.seq_len // n_seq
    seqs = [[int(t) for t in rng.integers(0, c.vocab_size, size=int(n))] for n in rng.integers(70, 90, size=n_seq)]
    g = gpu_model(c, ow)
    cpus = [O.Model(c, ow, "cpu") for _ in seqs]
    for t in range(max(len(s) for s in seqs)):
        live = [i for i, s in enumerate(seqs) if t < len(s)]
        got = g.decode_batch([seqs[i][t] for i in live], [t] * len(live), [i * room + t for i in live],
                             [i * room for i in live])
        if t % 16 == 15 or t + 1 == max(len(s) for s in seqs):
            for r, i in enumerate(live):
                want = cpus[i].forward(seqs[i][t], t)
                assert_bits_equal(got[r], want, f"decode_batch step {t} sequence {i}")
        else:
            for i in live:
                cpus[i].forward(seqs[i][t], t)


def test_decode_batch_split_attention_long_windows():
    # the batched two-launch attention (k_attn_softmax_v_rows) with eight
    # query heads per KV head over windows of 1500-1800 positions, two
    # sequences in one cache; compared with per-sequence forward() at the
    # end and every 300 steps
    c = O.Config(dim=256, hidden_dim=128, n_layers=1, n_heads=8, n_kv_heads=1, vocab_size=64, seq_len=3800,
                 rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=32)
    ow = gaussian_weights(c, "q8_0", seed=1800)
    rng = np.random.default_rng(18)
    room = c.seq_len // 2
    seqs = [[int(t) for t in rng.integers(0, c.vocab_size, size=n)] for n in (1500, 1800)]
    g = gpu_model(c, ow)
    cpus = [O.Model(c, ow, "cpu") for _ in seqs]
    n_max = max(len(x) for x in seqs)
    for t in range(n_max):
        live = [i for i, x in enumerate(seqs) if t < len(x)]
        got = g.decode_batch([seqs[i][t] for i in live], [t] * len(live), [i * room + t for i in live],
                             [i * room for i in live])
        check = t % 300 == 299 or any(t + 1 == len(seqs[i]) for i in live)
        for r, i in enumerate(live):
            want = cpus[i].forward(seqs[i][t], t)
            if check:
                assert_bits_equal(got[r], want, f"decode_batch step {t} sequence {i}")


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("dim,hidden", [(128, 256), (1024, 2048)])
def test_decode_at_fused_swiglu_widths(storage, dim, hidden):
    # widths where the fused decode step computes gate/up, SiLU * up and its
    # Q8 in one launch (64 <= dim <= 1024, hidden % 32 == 0): logits bitwise
    # against the cpu backend, both weight formats (FMA chain and the four
    # partial sums in the kernel's epilogue)
    c = O.Config(dim=dim, hidden_dim=hidden, n_layers=2, n_heads=dim // 64, n_kv_heads=dim // 128, vocab_size=128,
                 seq_len=64, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=64)
    ow = O.backends_weights(c, storage)
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    for pos, tok in enumerate(PROMPT):
        assert_bits_equal(gpu.forward(tok, pos), cpu.forward(tok, pos), f"{storage} {dim} pos {pos}")


@pytest.mark.parametrize("dim,hidden,n_tok", [(256, 3200, 200), (128, 96, 70), (128, 256, 9)])
def test_prefill_ffn_gate_up_silu_in_one_gemm(dim, hidden, n_tok):
    # Q8_0 prefill of 8+ rows: gate and up as one GEMM whose epilogue forms
    # SiLU(gate) * up and its Q8 blocks (fused schedule). 200 rows x 100
    # hidden blocks take its 128-row tiles, 70 and 9 rows its 64-row ones
    # (two row tiles, and one partly empty); logits bitwise against the cpu
    # backend
    c = O.Config(dim=dim, hidden_dim=hidden, n_layers=2, n_heads=dim // 64, n_kv_heads=dim // 128, vocab_size=128,
                 seq_len=256, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0", seed=hidden + n_tok)
    prompt = [(i * 11 + 5) % c.vocab_size for i in range(n_tok)]
    assert_bits_equal(gpu_model(c, ow).prefill(prompt, 0), O.Model(c, ow, "cpu").prefill(prompt, 0),
                      f"{dim}x{hidden}, {n_tok} rows")


@pytest.mark.parametrize("n_kv,n1,n2", [(32, 100, 90), (8, 200, 50)])
def test_prefill_qkv_rope_kv_write_in_one_gemm(n_kv, n1, n2):
    # the 1.7B attention width (dim 2048, head_dim 64): prefills whose q/k/v
    # launch takes the 64-row tiles run RoPE and kv_write as the GEMM's
    # epilogue (100 and 90 rows at kv_mul 1, 200 rows at kv_mul 4; the
    # 50-row continuation takes the separate launches), and their down
    # projections run chain-split (65-256 rows at dim 2048), the planes summed
    # by the next layer's norm and by the final residual add; a first prompt,
    # a continuation at the next positions (reading the first prompt's keys
    # and values from the cache), then two decode steps; logits bitwise
    # against the cpu backend at each stage
    c = O.Config(dim=2048, hidden_dim=256, n_layers=2, n_heads=32, n_kv_heads=n_kv, vocab_size=64, seq_len=256,
                 rms_eps=1e-5, rope_theta=130_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0", seed=170 + n_kv, norms="uniform")
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    p1 = [(i * 13 + 1) % c.vocab_size for i in range(n1)]
    p2 = [(i * 5 + 7) % c.vocab_size for i in range(n2)]
    assert_bits_equal(gpu.prefill(p1, 0), cpu.prefill(p1, 0), "first prompt")
    assert_bits_equal(gpu.prefill(p2, n1), cpu.prefill(p2, n1), "continuation")
    for i, tok in enumerate([3, 9]):
        assert_bits_equal(gpu.forward(tok, n1 + n2 + i), cpu.forward(tok, n1 + n2 + i), f"decode {i}")


def test_multi_tile_shapes():
    # tests/backends.rs:436-481: a 70-row prompt against 256-wide projections
    c = O.Config(dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=128, seq_len=128,
                 rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=32)
    prompt = [(i * 7 + 3) % c.vocab_size for i in range(70)]
    for storage in ["q8_0", "q8_0x4"]:
        ow = O.backends_weights(c, storage)
        assert_bits_equal(gpu_model(c, ow).prefill(prompt, 0), O.Model(c, ow, "cpu").prefill(prompt, 0), storage)


def test_interleaved_rope_model():
    c = O.backends_config()
    c.rope_interleaved = True
    ow = O.backends_weights(c, "q8_0x4")
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    for pos, tok in enumerate(PROMPT):
        assert_bits_equal(gpu.forward(tok, pos), cpu.forward(tok, pos), f"pos {pos}")


@pytest.mark.parametrize("mask", [[True, True], [False, False], [False, True]])
@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_lfm2_matches_the_cpu_backend(mask, storage):
    # lfm2.rs:794-824 and :871-940, held to bit equality
    c = O.lfm2_config()
    ow = O.lfm2_weights(c, mask, storage)
    gpu = gpu_model(c, ow, lfm2=True)
    cpu = O.Model(c, ow, "cpu", lfm2=True)
    for pos, tok in enumerate(PROMPT):
        assert_bits_equal(gpu.forward(tok, pos), cpu.forward(tok, pos), f"{mask} pos {pos}")
    got = gpu_model(c, ow, lfm2=True).prefill(PROMPT, 0)
    want = O.Model(c, ow, "cpu", lfm2=True).prefill(PROMPT, 0)
    assert_bits_equal(got, want, f"{mask} prefill")


def _oracle_greedy(model, token, pos, n):
    out = []
    for i in range(n):
        logits = model.forward(token, pos + i)
        token = O.argmax(logits)
        out.append(token)
    return out


@pytest.mark.parametrize("use_graph", [False, True])
def test_greedy_decode_matches_the_oracle(use_graph):
    c = O.backends_config()
    ow = O.backends_weights(c, "q8_0x4")
    gpu = gpu_model(c, ow)
    gpu.prefill(PROMPT, 0)
    got = gpu.generate_greedy(7, len(PROMPT), 40, use_graph=use_graph)
    cpu = O.Model(c, ow, "cpu")
    cpu.prefill(PROMPT, 0)
    assert list(got) == _oracle_greedy(cpu, 7, len(PROMPT), 40)


@pytest.mark.parametrize("n_heads,n_kv,hs,ctx", [(2, 1, 64, 1100), (8, 8, 32, 300), (8, 2, 128, 300),
                                                 (8, 1, 64, 200), (16, 4, 64, 150), (15, 5, 64, 1000),
                                                 (6, 2, 32, 1020), (6, 2, 64, 1500), (2, 2, 64, 2100)])
def test_split_decode_attention_windows(n_heads, n_kv, hs, ctx):
    # The fused decode step's two-launch attention (k_attn_scores +
    # k_attn_softmax_v) for head groups 2, 1, 4, 8, 4, 3, 3, 3 and 1 and head
    # sizes 32-128, after a long prefill, up to windows of 2100+ positions
    # (the softmax launch's LDS holds its scores, V slice and product table
    # up to about 2000 positions at three query heads per KV head).
    c = O.Config(dim=n_heads * hs, hidden_dim=128, n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, vocab_size=64,
                 seq_len=ctx + 4, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=hs)
    ow = gaussian_weights(c, "q8_0", seed=ctx + hs)
    prompt = [(i * 7 + 3) % c.vocab_size for i in range(ctx)]
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    assert_bits_equal(gpu.prefill(prompt, 0), cpu.prefill(prompt, 0), "prefill")
    for t in range(3):
        assert_bits_equal(gpu.forward(5 + t, ctx + t), cpu.forward(5 + t, ctx + t), f"decode at {ctx + t}")


@pytest.mark.parametrize("n_heads,n_kv,hs,ctx", [(6, 2, 64, 3000), (8, 4, 128, 3500), (4, 2, 128, 4000),
                                                 (8, 1, 64, 3000), (4, 2, 64, 5000), (6, 2, 64, 6000)])
def test_split_decode_attention_in_passes(n_heads, n_kv, hs, ctx):
    # decode windows whose V slice and product table do not fit the LDS in
    # one piece beside the score rows: the softmax+V launch runs them in 2
    # (G = 3 and 2) up to 8 (G = 8) passes, the chains continuing across
    # passes; past 4096 positions the softmax sums run on one lane and the
    # chunk maxima 64 apart per lane; the cache is filled directly, then two
    # decode steps
    c = O.Config(dim=n_heads * hs, hidden_dim=128, n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, vocab_size=64,
                 seq_len=ctx + 4, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=hs)
    ow = gaussian_weights(c, "q8_0", seed=ctx + hs + n_kv)
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    rng = np.random.default_rng(ctx + n_heads)
    kv = n_kv * hs
    keys = rng.normal(size=ctx * kv).astype(np.float32)
    vals = rng.normal(size=ctx * kv).astype(np.float32)
    gpu.backend.kv_upload(0, 0, keys)
    gpu.backend.kv_upload(1, 0, vals)
    cpu.kv_upload(0, 0, keys)
    cpu.kv_upload(1, 0, vals)
    for t in range(2):
        assert_bits_equal(gpu.forward(5 + t, ctx + t), cpu.forward(5 + t, ctx + t), f"decode at {ctx + t}")


def test_greedy_256_tokens_at_360m_width():
    # SmolLM2-360M widths (dim 960, 15/5 heads, hd 64, hidden 2560, theta 1e5)
    # with 2 layers and an 8192-token vocabulary so the oracle finishes fast:
    # 256 greedy tokens must be identical.
    c = O.Config(dim=960, hidden_dim=2560, n_layers=2, n_heads=15, n_kv_heads=5, vocab_size=8192, seq_len=512,
                 rms_eps=1e-5, rope_theta=100_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0x4", seed=360)
    prompt = list(np.random.default_rng(1).integers(0, c.vocab_size, size=16))
    gpu = gpu_model(c, ow)
    gpu.prefill(prompt, 0)
    got = gpu.generate_greedy(int(prompt[-1]), len(prompt), 256, use_graph=True)
    cpu = O.Model(c, ow, "cpu")
    cpu.prefill(prompt, 0)
    want = _oracle_greedy(cpu, int(prompt[-1]), len(prompt), 256)
    assert list(got) == want


@pytest.mark.parametrize("n_heads,n_kv,hs,storage", [(4, 2, 128, "q8_0"), (4, 4, 64, "q8_0x4"), (6, 2, 64, "q8_0")])
def test_long_prefill_attention_on_the_matrix_core(n_heads, n_kv, hs, storage):
    # Windows of 1024+ positions take the three-launch matrix-core attention
    # (k_attn_mx_scores / k_attn_softmax_att / k_attn_mx_v: the score and V
    # chains as exact f32 MFMA), head groups 2, 1 and 3 (run as 1): a
    # 1100-token pass (causal windows from 1 to 1100 in 32-pair blocks), a
    # 150-token chunk over the cache, then two decode steps.
    c = O.Config(dim=n_heads * hs, hidden_dim=128, n_layers=1, n_heads=n_heads, n_kv_heads=n_kv, vocab_size=64,
                 seq_len=1280, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=hs)
    ow = gaussian_weights(c, storage, seed=hs + n_heads)
    prompt = [(i * 7 + 3) % c.vocab_size for i in range(1250)]
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    assert_bits_equal(gpu.prefill(prompt[:1100], 0), cpu.prefill(prompt[:1100], 0), "prefill 1100")
    assert_bits_equal(gpu.prefill(prompt[1100:], 1100), cpu.prefill(prompt[1100:], 1100), "chunk at 1100")
    for t in range(2):
        assert_bits_equal(gpu.forward(9 + t, 1250 + t), cpu.forward(9 + t, 1250 + t), f"decode at {1250 + t}")


@pytest.mark.parametrize("n_heads,n_kv,interleaved", [(16, 8, False), (24, 8, True)])
def test_long_prefill_with_qk_norm(n_heads, n_kv, interleaved):
    # q/k norms + RoPE + kv_write in one launch at 4 lanes per head item, the
    # form a prefill of 32768 or more (row, head) items takes (1100 rows x
    # 32 or 40 items of q, k and v): two layers, so every row's layer-1 q
    # (through its attention output) reaches the layer-2 cache that the
    # decode steps read, and every row's layer-1 k through the layer-1 cache
    c = O.Config(dim=n_heads * 32, hidden_dim=128, n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, vocab_size=64,
                 seq_len=1200, rms_eps=1e-6, rope_theta=1_000_000.0, rope_interleaved=interleaved, head_dim=32)
    ow = gaussian_weights(c, "q8_0", seed=n_heads + 7, qk_norm=True, norms="uniform")
    prompt = [(i * 5 + 1) % c.vocab_size for i in range(1150)]
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    assert_bits_equal(gpu.prefill(prompt[:1100], 0), cpu.prefill(prompt[:1100], 0), "prefill 1100")
    assert_bits_equal(gpu.prefill(prompt[1100:], 1100), cpu.prefill(prompt[1100:], 1100), "chunk at 1100")
    for t in range(2):
        assert_bits_equal(gpu.forward(9 + t, 1150 + t), cpu.forward(9 + t, 1150 + t), f"decode at {1150 + t}")


@pytest.mark.parametrize("n_heads,n_kv,hs,interleaved,storage",
                         [(16, 8, 128, False, "q8_0x4"), (6, 2, 64, True, "q8_0"), (8, 8, 64, False, "q8_0x4")])
def test_decode_with_qk_norm_in_the_scores_launch(n_heads, n_kv, hs, interleaved, storage):
    # the per-head q/k RMSNorm runs inside the decode scores launch: each
    # 64-row chunk's workgroup normalizes its query heads and the new key
    # before the rotation; eager steps, then a captured greedy generation,
    # over windows across 64-row chunks
    c = O.Config(dim=n_heads * hs, hidden_dim=128, n_layers=2, n_heads=n_heads, n_kv_heads=n_kv, vocab_size=64,
                 seq_len=400, rms_eps=1e-6, rope_theta=1_000_000.0, rope_interleaved=interleaved, head_dim=hs)
    ow = gaussian_weights(c, storage, seed=hs + n_heads, qk_norm=True, norms="uniform")
    prompt = [(i * 7 + 2) % c.vocab_size for i in range(130)]
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    assert_bits_equal(gpu.prefill(prompt, 0), cpu.prefill(prompt, 0), "prefill")
    for t in range(3):
        p = len(prompt) + t
        assert_bits_equal(gpu.forward(5 + t, p), cpu.forward(5 + t, p), f"decode at {p}")
    pos = len(prompt) + 3
    got = gpu.generate_greedy(11, pos, 40, use_graph=True)
    assert list(got) == _oracle_greedy(cpu, 11, pos, 40)


def test_greedy_graph_per_window_bucket():
    # The captured step is sized for a window bucket (a power of two from 512
    # covering the generation): three query heads per KV head on a 4100-slot
    # context, where the whole-context step cannot take the split attention
    # but the 512 and 1024 buckets do. Generations that stay in the captured
    # bucket reuse its graph; one that needs more recaptures it.
    c = O.Config(dim=384, hidden_dim=256, n_layers=1, n_heads=6, n_kv_heads=2, vocab_size=64, seq_len=4100,
                 rms_eps=1e-5, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0x4", seed=77)
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    prompt = [(i * 5 + 1) % c.vocab_size for i in range(16)]
    assert_bits_equal(gpu.prefill(prompt, 0), cpu.prefill(prompt, 0), "prefill")
    tok, pos = 3, len(prompt)
    for n in (40, 500, 30):  # windows to 56 (bucket 512), to 556 (recaptured at 1024), to 586 (kept)
        got = gpu.generate_greedy(tok, pos, n, use_graph=True)
        want = _oracle_greedy(cpu, tok, pos, n)
        assert list(got) == want, f"{n} steps from {pos}"
        tok, pos = want[-1], pos + n


def test_greedy_graph_past_the_split_attention_range():
    # a window past 2048 positions at three query heads per KV head: the
    # 4096 bucket (the whole context here) takes the general attention
    c = O.Config(dim=384, hidden_dim=256, n_layers=1, n_heads=6, n_kv_heads=2, vocab_size=64, seq_len=4100,
                 rms_eps=1e-5, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=64)
    ow = gaussian_weights(c, "q8_0x4", seed=78)
    gpu, cpu = gpu_model(c, ow), O.Model(c, ow, "cpu")
    prompt = [(i * 7 + 2) % c.vocab_size for i in range(2040)]
    assert_bits_equal(gpu.prefill(prompt, 0), cpu.prefill(prompt, 0), "prefill")
    got = gpu.generate_greedy(5, len(prompt), 60, use_graph=True)
    assert list(got) == _oracle_greedy(cpu, 5, len(prompt), 60)
