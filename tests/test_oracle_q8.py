"""Pins for the oracle's Q8 arithmetic (CPU only).

Each test either ports one of the reference's own unit tests (cited), or
checks the restatement against something independent of it: closed forms,
numpy's IEEE float16 conversion, int64 brute force, float64 sums.
"""

import numpy as np
import pytest

import oracle as O


def random(n, seed):
    """ops/mod.rs:49-60: the reference's LCG in [-0.5, 0.5)."""
    return O.lcg_fill(n, seed)


# ---- ports of src/ops/mod.rs tests ------------------------------------------

def test_q8_quantization_error_is_half_a_step():
    # ops/mod.rs:557-572
    for seed in range(8):
        x = random(96, 100 + seed)
        q, s, _ = O.quantize(x)
        for b, scale in enumerate(s):
            restored = q[b * 32:(b + 1) * 32].astype(np.float32) * scale
            assert np.all(np.abs(restored - x[b * 32:(b + 1) * 32]) <= scale / 2 + 1e-6)


def test_q8_is_exact_on_step_multiples():
    # ops/mod.rs:577-597 (known answer: scale 1/128 round-trips exactly)
    step = np.float32(1.0 / 128.0)
    vals = []
    for _ in range(2):
        for lane in range(32):
            k = 127.0 if lane == 0 else lane - 16.0
            vals.append(np.float32(k) * step)
    vals = np.array(vals, np.float32)
    q, s, _ = O.quantize(vals)
    assert np.all(s == step)
    for b in range(2):
        restored = q[b * 32:(b + 1) * 32].astype(np.float32) * s[b]
        assert np.array_equal(restored, vals[b * 32:(b + 1) * 32])


def test_q8_dot_tracks_f32_dot():
    # ops/mod.rs:616-627
    n = 512
    a = np.array([((i % 7) + 1.0) * 0.1 for i in range(n)], np.float32)
    b = np.array([((i % 5) + 1.0) * 0.2 for i in range(n)], np.float32)
    want = O.dot_scalar(a, b)
    qa, sa, _ = O.quantize(a)
    qb, sb, _ = O.quantize(b)
    got = O.dot_q8_0_scalar(qa, sa, qb, sb)
    assert abs(got - want) <= 0.03 * abs(want)


def test_q8_gemv_tracks_f32_gemv():
    # ops/mod.rs:630-645
    out_dim, in_dim = 16, 128
    w = np.array([((i % 11) + 1.0) * 0.05 for i in range(out_dim * in_dim)], np.float32).reshape(out_dim, in_dim)
    x = np.array([((i % 7) + 1.0) * 0.1 for i in range(in_dim)], np.float32)
    ref = O.Matrix(w, "f32").gemv(x)
    quant = O.Matrix(w, "q8_0").gemv(x)
    assert np.all(np.abs(quant - ref) <= 0.05 * np.abs(ref))


def test_q8_requires_block_aligned_rows():
    # ops/mod.rs:648-651
    assert O.Matrix.try_new(np.zeros((2, 5), np.float32), "q8_0") is None
    assert O.Matrix.try_new(np.zeros((2, 32), np.float32), "q8_0") is not None


def test_q8_matrix_reads_rows():
    # ops/mod.rs:654-660
    m = O.Matrix(np.zeros((2, 64), np.float32), "q8_0")
    assert m.decode_row(0).size == 64
    assert np.all(m.decode_row(1) == 0.0)


def test_q8x4_repacked_rows_match_plain_q8_rows():
    # ops/mod.rs:663-676
    for out_dim, in_dim in [(4, 32), (8, 64), (16, 128), (12, 96)]:
        w = random(out_dim * in_dim, 711).reshape(out_dim, in_dim)
        x = random(in_dim, 712)
        plain = O.Matrix(w, "q8_0").gemv(x)
        packed = O.Matrix(w, "q8_0x4").gemv(x)
        assert np.all(np.abs(packed - plain) <= 5e-4 * (1 + np.abs(plain)))


def test_q8x4_rejects_unaligned_shapes():
    # ops/mod.rs:679-683
    assert O.Matrix.try_new(np.zeros((6, 32), np.float32), "q8_0x4") is None
    assert O.Matrix.try_new(np.zeros((8, 30), np.float32), "q8_0x4") is None
    assert O.Matrix.try_new(np.zeros((8, 32), np.float32), "q8_0x4") is not None


def _dense_data(out_dim, in_dim):
    return np.array([((i * 17 % 251) - 125.0) / 137.0 for i in range(out_dim * in_dim)],
                    np.float32).reshape(out_dim, in_dim)


def test_q8x4_to_row_major_matches_decode_row():
    # ops/mod.rs:689-712
    for out_dim, in_dim in [(4, 32), (8, 64), (16, 128)]:
        m = O.Matrix(_dense_data(out_dim, in_dim), "q8_0x4")
        q, s = m.to_row_major()
        nb = in_dim // 32
        for r in range(out_dim):
            row = m.decode_row(r)
            back = q[r * in_dim:(r + 1) * in_dim].astype(np.float32) * np.repeat(s[r * nb:(r + 1) * nb], 32)
            assert np.all(np.abs(back - row) <= 1e-6)


def test_q8x4_decodes_each_row_to_the_plain_quantization():
    # ops/mod.rs:715-732
    d = _dense_data(8, 64)
    a = O.Matrix(d, "q8_0x4")
    b = O.Matrix(d, "q8_0")
    for r in range(8):
        x, y = a.decode_row(r), b.decode_row(r)
        assert np.all(np.abs(x - y) <= 5e-4 * (1 + np.abs(y)))


def test_bf16_bits_round_to_the_stored_width():
    # ops/mod.rs:753-763 (through the matrix cast)
    for v in [0.0, 1.0, -1.0, 0.1, 0.123456, 1e-3, -1234.5, 1e20]:
        m = O.Matrix(np.array([[v]], np.float32), "bf16")
        back = m.decode_row(0)[0]
        assert abs(back - np.float32(v)) <= abs(v) * 0.0039 + np.finfo(np.float32).tiny


# ---- independent pins ---------------------------------------------------------

def test_f16_bits_match_ieee_rne_over_a_sweep():
    # quant.rs:722-758 against numpy's IEEE binary16 conversion (round to
    # nearest even), over normals, subnormals, ties, overflow and specials.
    rng = np.random.default_rng(0)
    bits = np.concatenate([
        rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32),
        # every f32 whose 13 dropped mantissa bits are exactly half (ties)
        (rng.integers(0, 2**19, 20_000, dtype=np.uint64).astype(np.uint32) << 13) | np.uint32(0x1000),
        np.arange(0x33000000, 0x38800000, 997, dtype=np.uint32),  # f16 subnormal range
        np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x477fe000, 0x477ff000, 0x47800000], np.uint32),
    ])
    vals = bits.view(np.float32)
    finite = np.isfinite(vals)
    want = vals[finite].astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_bits(v) for v in vals[finite]], np.uint16)
    assert np.array_equal(got, want)
    # NaN payloads: sign | 0x7c00 | 0x0200 (quant.rs:727-729)
    nan = np.array([0x7fc00001, 0xffa00000], np.uint32).view(np.float32)
    assert O.f32_to_f16_bits(nan[0]) == 0x7e00
    assert O.f32_to_f16_bits(nan[1]) == 0xfe00


def test_f16_scale_widening_closed_form_all_codes():
    # quant.rs:764-769: sign | (exp+112)<<23 | mant<<13 for all 65536 codes.
    # For exp in 1..30 this equals IEEE widening; exp == 0 is the reference's
    # quirk (a zero scale widens to 2^-15).
    for b in range(0, 65536, 1):
        sign = (b >> 15) << 31
        e = (b >> 10) & 0x1F
        m = b & 0x3FF
        want = np.array([sign | ((e + 112) << 23) | (m << 13)], np.uint32).view(np.float32)[0]
        got = np.float32(O.f16_scale_to_f32(b))
        assert got.view(np.uint32) == want.view(np.uint32)
        if 1 <= e <= 30:
            assert got == np.array([b], np.uint16).view(np.float16)[0].astype(np.float32)
    assert O.f16_scale_to_f32(0) == 2.0 ** -15


def test_quantize_special_cases():
    # all-zero block -> d = 0, q = 0; the amax element -> +-127; NaN -> 0
    q, s, h = O.quantize(np.zeros(32, np.float32))
    assert s[0] == 0.0 and h[0] == 0 and np.all(q == 0)
    x = np.linspace(-1, 0.5, 32).astype(np.float32)
    q, s, _ = O.quantize(x)
    assert q[0] == -127 and s[0] == np.float32(1.0) / np.float32(127.0)
    # exact .5 ties round away from zero: amax 127 -> d = 1, inv = 1
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -2.5, 0.5
    q, s, _ = O.quantize(x)
    assert s[0] == 1.0 and list(q[:4]) == [127, 3, -3, 1]
    x[5] = np.nan
    q, s, _ = O.quantize(x)
    assert q[5] == 0 and s[0] == 1.0  # NaN ignored by the amax fold
    # partial tail block is zero-padded (quant.rs:832,835)
    q, s, _ = O.quantize(np.ones(40, np.float32))
    assert q.size == 64 and np.all(q[40:] == 0) and s.size == 2


def test_quantize_matches_closed_form_brute_force():
    rng = np.random.default_rng(1)
    x = rng.normal(size=4096).astype(np.float32)
    q, s, h = O.quantize(x)
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(s, d)
    inv = np.where(d > 0, np.float32(1.0) / d, np.float32(0)).astype(np.float32)
    t = (xb * inv[:, None]).astype(np.float32)
    want = np.clip(np.sign(t) * np.floor(np.abs(t) + np.float32(0.5)), -127, 127).astype(np.int8)
    assert np.array_equal(q.reshape(-1, 32), want)
    assert np.array_equal(h, d.astype(np.float16).view(np.uint16))


def test_block_dots_are_exact_integers():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, size=(12, 256)).astype(np.float32)
    for storage in ["q8_0", "q8_0x4"]:
        m = O.Matrix(w, storage)
        wq, _ = m.to_row_major()
        xq = rng.integers(-127, 128, size=(3, 256)).astype(np.int8)
        got = m.block_dots(xq)
        want = np.einsum("rbi,nbi->rnb", xq.reshape(3, 8, 32).astype(np.int64),
                         wq.reshape(12, 8, 32).astype(np.int64))
        assert np.array_equal(got, want)


def _a8_epilogue(isum, sa, sb):
    """dot.rs:34-45 in float32 numpy: t[b&3] += (sa*sb)*f32(isum)."""
    t = [np.float32(0)] * 4
    for b in range(isum.size):
        t[b & 3] = np.float32(t[b & 3] + np.float32(np.float32(sa[b] * sb[b]) * np.float32(isum[b])))
    return np.float32(np.float32(np.float32(t[0] + t[1]) + t[2]) + t[3])


def test_q8_0_gemv_order_and_float64_bound():
    rng = np.random.default_rng(3)
    out_dim, in_dim = 24, 576
    w = rng.normal(0, 0.02, size=(out_dim, in_dim)).astype(np.float32)
    x = rng.normal(size=in_dim).astype(np.float32)
    m = O.Matrix(w, "q8_0")
    got = m.project_cpu(x)[0]
    wq, ws = m.q8_0_data()
    xq, xs, _ = O.quantize(x)
    isum = m.block_dots(xq)[0]
    nb = in_dim // 32
    for n in range(out_dim):
        sa = ws[n * nb:(n + 1) * nb]
        assert got[n] == _a8_epilogue(isum[n], sa, xs)
        exact = float(np.sum(sa.astype(np.float64) * xs.astype(np.float64) * isum[n].astype(np.float64)))
        assert abs(got[n] - exact) <= 1e-5 * (1 + abs(exact))


def test_q8_0x4_gemm_order_and_float64_bound():
    # quant.rs:268-291: slot = fma(f32(isum), f16w(ws)*f16w(xs), slot)
    rng = np.random.default_rng(4)
    rows, out_dim, in_dim = 3, 16, 960
    w = rng.normal(0, 0.02, size=(out_dim, in_dim)).astype(np.float32)
    x = rng.normal(size=(rows, in_dim)).astype(np.float32)
    m = O.Matrix(w, "q8_0x4")
    got = m.project_cpu(x)
    _, wsf = m.to_row_major()
    nb = in_dim // 32
    for r in range(rows):
        xq, _, xh = O.quantize(x[r])
        isum = m.block_dots(xq)[0]
        xs = np.array([O.f16_scale_to_f32(b) for b in xh], np.float32)
        for n in range(out_dim):
            slot = np.float32(0)
            for b in range(nb):
                ws = np.float32(wsf[n * nb + b] * xs[b])
                slot = np.float32(np.float64(isum[n, b]) * np.float64(ws) + np.float64(slot))
            assert got[r, n] == slot
            exact = float(np.sum(wsf[n * nb:(n + 1) * nb].astype(np.float64) * xs.astype(np.float64)
                                 * isum[n].astype(np.float64)))
            assert abs(got[r, n] - exact) <= 1e-5 * (1 + abs(exact))


def test_q8_0x4_logits_requantize_identity():
    # quant.rs:223-236 (x86): re-quantizing a decoded Q8_0x4 row gives back the
    # same quants and the widened f16 scale, so logits equal the Q8_0 dot
    # with f16-widened weight scales.
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, size=(64, 960)).astype(np.float32)
    w[3, 64:96] = 0.0  # an all-zero block
    m = O.Matrix(w, "q8_0x4")
    x = rng.normal(size=960).astype(np.float32)
    got = m.logits_cpu(x)
    wq, wsf = m.to_row_major()
    xq, xs, _ = O.quantize(x)
    nb = 30
    for n in range(64):
        want = O.dot_q8_0_scalar(wq[n * 960:(n + 1) * 960], wsf[n * nb:(n + 1) * nb], xq, xs)
        assert got[n] == np.float32(want)


def test_argmax_keeps_the_last_maximum():
    # generate.rs:70-77: Iterator::max_by(total_cmp) returns the last maximum
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 2
    assert O.argmax([0.0, -0.0]) == 0  # +0 > -0 under total_cmp
    assert O.argmax([-0.0, 0.0, -0.0]) == 1
    assert O.argmax([float("-inf"), -1.0]) == 1


def test_softmax_known_values():
    # ops/mod.rs softmax KAT: softmax([1, 2, 3]) and shift invariance
    got = O.softmax([1.0, 2.0, 3.0])
    e = np.exp(np.array([-2.0, -1.0, 0.0]))
    assert np.allclose(got, e / e.sum(), rtol=1e-6)
    big = O.softmax([1000.0, 1001.0, 1002.0])
    assert np.allclose(big, got, rtol=1e-6)
