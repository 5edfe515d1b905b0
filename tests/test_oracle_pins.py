"""Known-answer pins for the oracle's non-Q8 ops: RoPE, RMSNorm, qk_norm,
SiLU, the depthwise conv and attention (cpu.rs:557-710, reference.rs:160-257).

Each expected value is either a hand computation the reference's own tests
hold (metal.rs:2239-2280 for the conv) or a closed form evaluated in float64
(Python's math module), never the oracle's f32 expression retyped. The inputs
are chosen so that a plausible slip fails a check: a flipped sine sign, the
wrong sign of the RoPE frequency exponent, a per-width instead of per-head
frequency index, eps dropped or added outside the square root, a sum instead
of a mean, a missing weight, a missing 1/sqrt(head_size), the wrong KV head
under grouping, or a window that includes a position it should skip.

Both oracle backends are checked: the cpu backend (cpu.rs) and the reference
backend, whose rms_norm, qk_norm and rope are a separate transcription of
reference.rs, so that their bitwise agreement on random inputs below compares
two restatements of two reference files.
"""

import math

import numpy as np
import pytest

import oracle as O

BACKENDS = ["cpu", "reference"]


def close(got, want, rel=2e-7, abs_=1e-7):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    lim = abs_ + rel * np.abs(want)
    assert np.all(err <= lim), f"got {got.tolist()} want {want.tolist()} (max err {err.max():.3g})"


def run_rope(name, q, k, qw, kvw, positions, hs, theta, interleaved):
    b = O.Backend(name)
    qb, kb = b.upload(q), b.upload(k)
    b.rope(qb, kb, qw, kvw, len(positions), positions, hs, theta, interleaved)
    return b.read(qb, len(q)), b.read(kb, len(k))


# ---- RoPE (cpu.rs:664-705, reference.rs:209-257) ---------------------------


@pytest.mark.parametrize("name", BACKENDS)
@pytest.mark.parametrize("pos", [1, 3])
def test_rope_half_rotates_pair_i_by_pos_theta_pow_minus_2i_over_d(name, pos):
    hs, theta = 8, 10_000.0
    half = hs // 2
    # head 0: lo = 1, hi = 0 (so lo' = cos a, hi' = +sin a);
    # head 1: lo = 0, hi = 1 (so lo' = -sin a, hi' = cos a) -- the sign case
    q = np.zeros(2 * hs, np.float32)
    q[:half] = 1.0
    q[hs + half:] = 1.0
    k = q[:hs].copy()
    gq, gk = run_rope(name, q, k, 2 * hs, hs, [pos], hs, theta, False)
    angles = [pos * theta ** (-2.0 * i / hs) for i in range(half)]  # pos, pos/10, pos/100, pos/1000
    want_q = np.zeros(2 * hs)
    for i, a in enumerate(angles):
        want_q[i], want_q[i + half] = math.cos(a), math.sin(a)
        want_q[hs + i], want_q[hs + i + half] = -math.sin(a), math.cos(a)
    close(gq, want_q)
    close(gk, want_q[:hs])  # k rotates exactly like q's head 0


@pytest.mark.parametrize("name", BACKENDS)
def test_rope_interleaved_rotates_adjacent_pairs_per_head(name):
    hs, theta, pos = 8, 10_000.0, 1
    # two heads: the frequency index restarts per head (i % head_size)
    q = np.tile(np.array([1.0, 0.0], np.float32), hs)          # 16 values
    q[hs:] = np.tile(np.array([0.0, 1.0], np.float32), hs // 2)  # head 1: the sign case
    k = np.tile(np.array([1.0, 0.0], np.float32), hs)
    # kv width 8 < q width 16: only k's pairs with i < 8 rotate
    gq, gk = run_rope(name, q, k, 2 * hs, hs, [pos], hs, theta, True)
    want_q = np.zeros(2 * hs)
    for j in range(hs // 2):
        a = pos * theta ** (-(2.0 * j) / hs)
        want_q[2 * j], want_q[2 * j + 1] = math.cos(a), math.sin(a)
        want_q[hs + 2 * j], want_q[hs + 2 * j + 1] = -math.sin(a), math.cos(a)
    close(gq, want_q)
    close(gk[:hs], want_q[:hs])
    assert np.array_equal(gk[hs:], k[hs:])


@pytest.mark.parametrize("name", BACKENDS)
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_position_zero_is_the_identity_bitwise(name, interleaved):
    rng = np.random.default_rng(3)
    q = rng.normal(size=32).astype(np.float32)
    k = rng.normal(size=16).astype(np.float32)
    gq, gk = run_rope(name, q, k, 32, 16, [0], 16, 1e6, interleaved)
    assert np.array_equal(gq.view(np.uint32), q.view(np.uint32))
    assert np.array_equal(gk.view(np.uint32), k.view(np.uint32))


@pytest.mark.parametrize("name", BACKENDS)
def test_rope_rows_take_their_own_positions(name):
    hs = 4
    q = np.array([1, 0, 0, 0] * 3, np.float32)
    k = q.copy()
    gq, _ = run_rope(name, q, k, hs, hs, [0, 2, 5], hs, 100.0, False)
    # pair 0 (frequency 1) of row r turns by exactly its position; pair 1 is zero
    for r, pos in enumerate([0, 2, 5]):
        close(gq[r * hs:(r + 1) * hs], [math.cos(pos), 0.0, math.sin(pos), 0.0], abs_=1e-6)


def test_rope_large_position_tracks_the_real_angle():
    # at pos 1000 the f32 angle is pos * f32(1/theta^(2i/d)): within a few
    # ulps of the real angle, so cos/sin agree with float64 to ~1e-4
    hs, theta, pos = 64, 1e5, 1000
    q = np.zeros(hs, np.float32)
    q[: hs // 2] = 1.0
    gq, _ = run_rope("cpu", q, q.copy(), hs, hs, [pos], hs, theta, False)
    for i in range(hs // 2):
        a = pos * theta ** (-2.0 * i / hs)
        assert abs(gq[i] - math.cos(a)) < 2e-4 and abs(gq[i + hs // 2] - math.sin(a)) < 2e-4, i


# ---- RMSNorm (cpu.rs:633-644, reference.rs:160-176) ------------------------


@pytest.mark.parametrize("name", BACKENDS)
def test_rms_norm_hand_computed_with_eps(name):
    b = O.Backend(name)
    # row 0: mean(x^2) = 12.5, + eps 1.0 = 13.5; row 1: mean = 7.5
    x = np.array([3.0, 4.0, 1.0, 2.0 * math.sqrt(3.5)], np.float32)
    w = np.array([2.0, 0.5], np.float32)
    xb, wb, ob = b.upload(x), b.upload(w), b.alloc(4)
    b.rms_norm(ob, xb, wb, 2, 2, 1.0)
    got = b.read(ob, 4)
    s0 = 1.0 / math.sqrt(12.5 + 1.0)
    ms1 = (1.0 + float(x[3]) ** 2) / 2.0
    s1 = 1.0 / math.sqrt(ms1 + 1.0)
    close(got, [2.0 * 3.0 * s0, 0.5 * 4.0 * s0, 2.0 * 1.0 * s1, 0.5 * float(x[3]) * s1])


@pytest.mark.parametrize("name", BACKENDS)
def test_rms_norm_small_eps(name):
    b = O.Backend(name)
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    xb, wb, ob = b.upload(x), b.upload(np.ones(4, np.float32)), b.alloc(4)
    b.rms_norm(ob, xb, wb, 1, 4, 1e-5)
    s = 1.0 / math.sqrt(30.0 / 4.0 + float(np.float32(1e-5)))
    close(b.read(ob, 4), [s, 2 * s, 3 * s, 4 * s])


# ---- qk_norm (cpu.rs:647-661, reference.rs:178-207) ------------------------


@pytest.mark.parametrize("name", BACKENDS)
def test_qk_norm_per_head_with_eps_and_weight(name):
    b = O.Backend(name)
    v = np.array([1, 1, 1, 1, 2, 2, 0, 0, 0, 0, 0, 3], np.float32)  # one row, three heads of 4
    w = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    vb, wb = b.upload(v), b.upload(w)
    b.qk_norm(vb, 1, 12, 4, wb, 0.5)
    got = b.read(vb, 12)
    want = []
    for h in range(3):
        head = [float(t) for t in v[4 * h:4 * h + 4]]
        s = 1.0 / math.sqrt(sum(t * t for t in head) / 4.0 + 0.5)
        want += [w[i] * s * head[i] for i in range(4)]
    close(got, want)


@pytest.mark.parametrize("name", BACKENDS)
def test_qk_norm_rows_and_heads(name):
    b = O.Backend(name)
    rng = np.random.default_rng(11)
    rows, heads, hs, eps = 3, 2, 8, 1e-6
    v = rng.normal(size=rows * heads * hs).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=hs).astype(np.float32)
    vb, wb = b.upload(v), b.upload(w)
    b.qk_norm(vb, rows, heads * hs, hs, wb, eps)
    got = b.read(vb, v.size).reshape(rows, heads, hs)
    vv = v.astype(np.float64).reshape(rows, heads, hs)
    want = w[None, None, :] * vv / np.sqrt(np.mean(vv * vv, axis=2, keepdims=True) + eps)
    close(got, want, rel=1e-6, abs_=1e-6)


# ---- SiLU (cpu.rs:708-710) ---------------------------------------------------


@pytest.mark.parametrize("name", BACKENDS)
def test_silu_mul_exact_values(name):
    b = O.Backend(name)
    g = np.array([0.0, 1.0, -1.0, 10.0, -10.0, 100.0, 2.0, 0.5], np.float32)
    u = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 3.0, -2.0], np.float32)
    gb, ub = b.upload(g), b.upload(u)
    b.silu_mul(gb, ub, 8)
    got = b.read(gb, 8)
    want = [float(x) / (1.0 + math.exp(-float(x))) * float(y) for x, y in zip(g, u)]
    # silu(1) = 0.7310585786300049, silu(-1) = -0.2689414213699951
    assert abs(want[1] - 0.7310585786300049) < 1e-15 and abs(want[2] + 0.2689414213699951) < 1e-15
    close(got, want)


def test_silu_far_negative():
    # x / (1 + exp(-x)) in f32: at -80, exp(80) = 5.5e34 is finite and the
    # result a tiny negative normal; at -100, exp(100) overflows to inf and
    # the quotient is exactly -0.0
    b = O.Backend("cpu")
    gb, ub = b.upload(np.array([-80.0, -100.0], np.float32)), b.upload(np.ones(2, np.float32))
    b.silu_mul(gb, ub, 2)
    got = b.read(gb, 2)
    close(got[:1], [-80.0 / (1.0 + math.exp(80.0))], rel=1e-6, abs_=0.0)
    assert got[1] == 0.0 and np.signbit(got[1])


# ---- the LFM2 depthwise conv (metal.rs:2239-2280) ----------------------------


@pytest.mark.parametrize("name", BACKENDS)
def test_conv_prefill_hand_computation(name):
    b = O.Backend(name)
    x = np.arange(1, 17, dtype=np.float32)
    kw = np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, 1, 1, 1], np.float32)
    xb, kb, ob = b.upload(x), b.upload(kw), b.alloc(16)
    b.conv_prefill(ob, xb, kb, 4, 4, 3)
    got = b.read(ob, 16)
    # the reference's asserts (metal.rs:2256-2262)
    assert got[0] == 0.0 and got[4] == 0.0
    assert got[8] == x[0] and got[12] == x[4]
    assert got[3] == x[3] and got[15] == x[7] + x[11] + x[15]
    # the whole table by exact integer arithmetic: row r, lane i sees
    # x[r-2+j] through tap j, zero below row 0
    want = np.zeros(16)
    for r in range(4):
        for i in range(4):
            want[r * 4 + i] = sum(int(kw[i * 3 + j]) * int(x[(r - 2 + j) * 4 + i])
                                  for j in range(3) if r - 2 + j >= 0)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("name", BACKENDS)
def test_conv_decode_hand_computation_and_ring(name):
    b = O.Backend(name)
    kw = np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, 1, 1, 1], np.float32)
    kb = b.upload(kw)
    st = b.upload(np.array([10, 20, 30, 40, 50, 60, 70, 80], np.float32))
    xr = b.upload(np.ones(4, np.float32))
    orow = b.alloc(4)
    b.conv_decode(orow, xr, kb, st, 4, 3)
    got = b.read(orow, 4)
    assert got[0] == 10.0 and got[3] == 40.0 + 80.0 + 1.0  # metal.rs:2273-2274
    assert got[1] == 60.0 and got[2] == 1.0                # tap 1: ring row 1; tap 2: x
    assert b.read(st, 8).tolist() == [50, 60, 70, 80, 1, 1, 1, 1]


# ---- attention (cpu.rs:575-630) -----------------------------------------------


def attention_case(name, kc, vc, q, windows, n_heads, kv_mul, hs, kv_dim, seq_len):
    b = O.Backend(name, None, 1, kv_dim, seq_len)
    kb, vb = b.upload(kc.ravel()), b.upload(vc.ravel())
    n_rows = kc.shape[0]
    b.kv_write(0, list(range(n_rows)), kb, vb, n_rows)
    qb = b.upload(q)
    out = b.alloc(len(windows) * n_heads * hs)
    att = b.alloc(len(windows) * n_heads * seq_len)
    b.attention(qb, out, att, 0, windows, n_heads, kv_mul, hs, kv_dim, seq_len)
    return b.read(out, len(windows) * n_heads * hs)


def softmax_v(q, keys, values, hs):
    s = [sum(a * b for a, b in zip(q, k)) / math.sqrt(hs) for k in keys]
    m = max(s)
    e = [math.exp(t - m) for t in s]
    z = sum(e)
    return [sum(e[i] / z * values[i][d] for i in range(len(keys))) for d in range(hs)]


@pytest.mark.parametrize("name", BACKENDS)
def test_attention_two_positions_by_hand(name):
    kc = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    vc = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    got = attention_case(name, kc, vc, np.array([1.0, 0.0], np.float32), [(0, 1, 0, 0)], 1, 1, 2, 2, 4)
    p0 = 1.0 / (1.0 + math.exp(-1.0 / math.sqrt(2.0)))  # scores [1/sqrt 2, 0]
    close(got, [p0 * 1 + (1 - p0) * 3, p0 * 2 + (1 - p0) * 4])


def test_softmax_subtracts_the_maximum():
    # elementwise.rs:81-91 subtracts the row maximum before exp: scores near 1000
    # would overflow exp without it (e^1000 = inf in f32, inf / inf = NaN).
    got = O.softmax(np.array([1000.0, 1001.0, 999.0], np.float32))
    e = [math.exp(-1.0), 1.0, math.exp(-2.0)]
    close(got, [v / sum(e) for v in e], rel=1e-6, abs_=0.0)


@pytest.mark.parametrize("name", BACKENDS)
def test_attention_large_scores_by_hand(name):
    # q.k = 1000/sqrt 2 and 999/sqrt 2 after scaling: finite only when the
    # maximum is taken out first
    kc = np.array([[1000.0, 0.0], [999.0, 0.0]], np.float32)
    vc = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    got = attention_case(name, kc, vc, np.array([1.0, 0.0], np.float32), [(0, 1, 0, 0)], 1, 1, 2, 2, 4)
    # scores are rounded to f32 (dot * (1 / sqrt hs), cpu.rs:591-609): at 700
    # their ulp is 6e-5, so the hand computation takes the same roundings
    scale = np.float32(1.0) / np.sqrt(np.float32(2.0))
    d = float(np.float32(1000.0) * scale) - float(np.float32(999.0) * scale)
    p0 = 1.0 / (1.0 + math.exp(-d))
    close(got, [p0 * 1 + (1 - p0) * 3, p0 * 2 + (1 - p0) * 4], rel=1e-5, abs_=1e-6)


@pytest.mark.parametrize("name", BACKENDS)
def test_attention_grouped_heads_and_windows(name):
    # 4 cache rows, kv_dim 4 = two KV heads of 2; q has 4 heads (kv_mul 2):
    # heads 0,1 read KV head 0, heads 2,3 read KV head 1
    rng = np.random.default_rng(5)
    kc = rng.normal(size=(4, 4)).astype(np.float32)
    vc = rng.normal(size=(4, 4)).astype(np.float32)
    q = rng.normal(size=2 * 8).astype(np.float32)
    # row 0: own range 0..=2; row 1: shared [0,1) then own 2..=3 (skips position 1)
    windows = [(0, 2, 0, 0), (2, 3, 0, 1)]
    got = attention_case(name, kc, vc, q, windows, 4, 2, 2, 4, 8).reshape(2, 4, 2)
    for r, pos_list in enumerate([[0, 1, 2], [0, 2, 3]]):
        for h in range(4):
            kvh = h // 2
            keys = [[float(v) for v in kc[t, 2 * kvh:2 * kvh + 2]] for t in pos_list]
            vals = [[float(v) for v in vc[t, 2 * kvh:2 * kvh + 2]] for t in pos_list]
            qh = [float(v) for v in q[r * 8 + 2 * h: r * 8 + 2 * h + 2]]
            close(got[r, h], softmax_v(qh, keys, vals, 2), rel=1e-6, abs_=1e-6)


# ---- the two transcriptions agree bit for bit ------------------------------


@pytest.mark.parametrize("interleaved", [False, True])
def test_cpu_and_reference_transcriptions_agree_bitwise(interleaved):
    rng = np.random.default_rng(21)
    rows, hs, nq, nkv = 5, 16, 4, 2
    q = rng.normal(size=rows * nq * hs).astype(np.float32)
    k = rng.normal(size=rows * nkv * hs).astype(np.float32)
    x = rng.normal(size=rows * 48).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=48).astype(np.float32)
    outs = {}
    for name in BACKENDS:
        b = O.Backend(name)
        qb, kb = b.upload(q), b.upload(k)
        b.rope(qb, kb, nq * hs, nkv * hs, rows, [0, 1, 7, 100, 4095], hs, 1e4, interleaved)
        wq = b.upload(w[:hs])
        b.qk_norm(qb, rows, nq * hs, hs, wq, 1e-6)
        xb, wb, ob = b.upload(x), b.upload(w), b.alloc(x.size)
        b.rms_norm(ob, xb, wb, rows, 48, 1e-5)
        outs[name] = np.concatenate([b.read(qb, q.size), b.read(kb, k.size), b.read(ob, x.size)])
    assert np.array_equal(outs["cpu"].view(np.uint32), outs["reference"].view(np.uint32))


# ---- dot_scalar: four FMA chains (src/ops/dot.rs:350-366) -------------------
#
# The attention scores use this dot, on the CPU and (restated) on the GPU.
# Each case is worked by hand in f32 so that a plausible restatement mistake
# gives a different exact answer: a single left-to-right chain, separate
# multiply and add instead of mul_add, the chains joined in sequence instead
# of pairwise, or the tail summed on its own.


def test_dot_scalar_runs_four_chains_not_one():
    # chain 0: fma(1e8, 1, 0) = 1e8, fma(-1e8, 1, 1e8) = 0; chains 1-3: 1 + 1 = 2
    # -> (0 + 2) + (2 + 2) = 6. One chain: 1e8 + 1 = 1e8 (ulp 8) three times,
    # then -1e8 -> 0, then + 1 + 1 + 1 = 3.
    a = [1e8, 1, 1, 1, -1e8, 1, 1, 1]
    assert O.dot_scalar(a, np.ones(8)) == 6.0


def test_dot_scalar_fuses_the_multiply_add():
    # chain 0: fma(-1, 1 + 2^-11, 0) = -(1 + 2^-11), then
    # fma(1 + 2^-12, 1 + 2^-12, -(1 + 2^-11)) = exactly 2^-24. A separate
    # product rounds (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 (a tie) to even,
    # 1 + 2^-11, and the sum is 0.
    u, v = 1 + 2.0 ** -12, 1 + 2.0 ** -11
    a = [-1.0, 0, 0, 0, u, 0, 0, 0]
    b = [v, 0, 0, 0, u, 0, 0, 0]
    assert O.dot_scalar(a, b) == 2.0 ** -24


def test_dot_scalar_joins_the_chains_pairwise():
    # acc = [1, 1e8, -1e8, 1]: (1 + 1e8) + (-1e8 + 1) = 1e8 + -1e8 = 0;
    # in sequence ((1 + 1e8) - 1e8) + 1 = 1.
    assert O.dot_scalar([1.0, 1e8, -1e8, 1.0], np.ones(4)) == 0.0


def test_dot_scalar_continues_the_tail_from_the_joined_sum():
    # chains give 1e8; the tail: fma(-1e8, 1, 1e8) = 0, fma(1, 1, 0) = 1.
    # A tail summed apart (-1e8 + 1 = -1e8) and then added would give 0.
    assert O.dot_scalar([1e8, 0, 0, 0, -1e8, 1.0], np.ones(6)) == 1.0
