"""GPU checks of the premises the exact kernels rest on, and of the
matrix-core prefill attention at the op level.

* The f32 matrix instruction v_mfma_f32_32x32x1_2b_f32 computes every output
  as fmaf(a, b, c) of its operands (one nonzero product term). The prefill
  GEMM forms the scale products sa * sb with it (c = +0: the correctly
  rounded product), and the prefill attention runs the reference's score and
  V chains on it. Checked here against the host's fmaf on typical,
  subnormal, cancelling, overflowing and infinite operands.
* k_attn_mx_* (windows of 1024..4570 positions in the prefill layout): every
  row's output and probabilities against the oracle, several 32-pair blocks
  and a partial one, with and without a shared prefix, kv_mul 1, 2, 3, 4, 8
  and head size 64 and 128; and a V row holding an infinity just past a
  short window, which the reference never reads for that row.
* Contract checks of the debug entries (sizes, probe limits).
"""

import ctypes

import numpy as np
import pytest

import kernrt_amd as K
import oracle as O
from helpers import assert_bits_equal, product_matrix

pytestmark = pytest.mark.gpu

_libm = ctypes.CDLL("libm.so.6")
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]


@pytest.fixture(scope="module")
def hip():
    h = K.open("hip")
    yield h
    h.close()


def _operands(kind, rng, groups):
    """a, b [groups, 64] and c [groups, 32, 64] of one operand class."""
    a = rng.normal(size=(groups, 64)).astype(np.float32)
    b = rng.normal(size=(groups, 64)).astype(np.float32)
    c = rng.normal(size=(groups, 32, 64)).astype(np.float32)
    if kind == "product":  # the GEMM's use: scales >= 0 and c = +0
        a = np.abs(a) * np.float32(1e-2)
        b = np.abs(b) * np.float32(1e-3)
        c[:] = 0.0
    elif kind == "subnormal":  # products and sums below 2^-126
        a *= np.float32(1e-20)
        b *= np.float32(1e-19)
        c *= np.float32(1e-39)
        a[:, ::7] = np.float32(3e-45) * np.sign(a[:, ::7])  # subnormal operands as well
    elif kind == "cancel":  # c close to -a*b: the fused result keeps the rounding error
        return a, b, None
    elif kind == "overflow":
        a *= np.float32(1e19)
        b *= np.float32(1e19)
        c *= np.float32(1e37)
    elif kind == "inf":
        a[:, ::5] = np.inf
        a[:, 1::5] = -np.inf
        b = np.where(b == 0, np.float32(1.0), b)  # no inf * 0 (NaN payloads are not compared)
        c[:, ::3, :] = np.inf
        c[:, 1::3, :] = 0.0
        # keep inf + -inf out of the sums: +inf c only where the product is not -inf
    elif kind == "wide":  # arbitrary finite bit patterns
        bits = rng.integers(0, 1 << 32, size=(groups, 64), dtype=np.uint64).astype(np.uint32)
        a = bits.view(np.float32).copy()
        bits = rng.integers(0, 1 << 32, size=(groups, 64), dtype=np.uint64).astype(np.uint32)
        b = bits.view(np.float32).copy()
        bits = rng.integers(0, 1 << 32, size=(groups, 32, 64), dtype=np.uint64).astype(np.uint32)
        c = bits.view(np.float32).copy()
        for arr in (a, b, c):
            arr[~np.isfinite(arr)] = 1.0
    return a, b, c


def _expected(a, b, c):
    """fmaf of each output's operands: register 16 blk + j of lane l is
    element (8 (j / 4) + 4 (l / 32) + j % 4, l % 32) of block blk."""
    g = a.shape[0]
    out = np.empty_like(c)
    for gi in range(g):
        for v in range(32):
            blk, j = v // 16, v % 16
            for l in range(64):
                row = 8 * (j // 4) + 4 * (l // 32) + j % 4
                col = l % 32
                out[gi, v, l] = _libm.fmaf(float(a[gi, 32 * blk + row]), float(b[gi, 32 * blk + col]),
                                           float(c[gi, v, l]))
    return out


KINDS = ["typical", "product", "subnormal", "cancel", "overflow", "inf", "wide"]


@pytest.mark.parametrize("kind", KINDS)
def test_f32_matrix_instruction_is_fmaf(hip, kind):
    rng = np.random.default_rng(31 + KINDS.index(kind))  # a fixed seed per operand class
    groups = 6
    a, b, c = _operands(kind, rng, groups)
    if kind == "cancel":
        # c[v][l] = -(a*b) rounded to f32 for the output's own operands
        c = np.empty((groups, 32, 64), np.float32)
        for gi in range(groups):
            for v in range(32):
                blk, j = v // 16, v % 16
                for l in range(64):
                    row = 8 * (j // 4) + 4 * (l // 32) + j % 4
                    c[gi, v, l] = -(a[gi, 32 * blk + row] * b[gi, 32 * blk + l % 32])
    if kind == "inf":
        # no +inf c where the product is -inf, and no -inf product meeting a +inf c
        want_prod = _expected(a, b, np.zeros_like(c))
        c = np.where(np.isinf(want_prod) & np.isinf(c), np.float32(0.0), c)
    got = hip.dbg_mfma_f32(a, b, c)
    want = _expected(a, b, c)
    nan = np.isnan(want)
    assert not nan.any() or kind == "wide", "the operands were meant to avoid NaN"
    same = np.isnan(got) == nan
    assert same.all(), f"{kind}: NaN where the fused result is not (or the reverse)"
    g, w = got[~nan], want[~nan]
    # the sign of an exact zero result is not asserted: the chains start at
    # +0 and the scales are never negative, so none of them can tell
    zero = w == 0
    assert np.array_equal(g[zero], w[zero]), f"{kind}: a zero result is not zero"
    nz = ~zero
    assert np.array_equal(g[nz].view(np.uint32), w[nz].view(np.uint32)), (
        f"{kind}: {int((g[nz].view(np.uint32) != w[nz].view(np.uint32)).sum())} outputs differ from fmaf")


# ---- the matrix-core prefill attention at the op level -----------------------

def _mx_case(seq_len, n_heads, n_kv, hs, windows, seed, inf_slot=None):
    """As test_gpu_ops._attention_case, with windows long enough for the
    matrix-core path; `inf_slot` writes +inf into a few dims of that V row."""
    rng = np.random.default_rng(seed)
    emb = O.Matrix(rng.normal(0, 0.02, size=(8, 32)).astype(np.float32), "q8_0")
    ow = O.Weights(1)
    ow.set_embedding(emb)
    kv_dim = n_kv * hs
    hip = K.open("hip")
    hip.bind_handles(hip.upload_matrix(product_matrix(emb)), 0xFFFFFFFF, [{}])
    hip.prepare(None, K.KvSpec(1, kv_dim, seq_len))
    ob = O.Backend("cpu", ow, n_layers=1, kv_dim=kv_dim, seq_len=seq_len)
    slots = np.arange(seq_len)
    kk = rng.normal(size=seq_len * kv_dim).astype(np.float32)
    vv = rng.normal(size=seq_len * kv_dim).astype(np.float32)
    if inf_slot is not None:
        vv[inf_slot * kv_dim + 3: inf_slot * kv_dim + kv_dim: 7] = np.inf
    hip.kv_write(0, slots, hip.upload(kk), hip.upload(vv), seq_len)
    ob.kv_write(0, slots, ob.upload(kk), ob.upload(vv), seq_len)
    n = len(windows)
    width = n_heads * hs
    q = (rng.normal(size=n * width) * 0.5).astype(np.float32)
    spec = K.AttnSpec(n_heads, n_heads // n_kv, hs, kv_dim, seq_len)
    go, ga = hip.alloc(n * width), hip.alloc(n * n_heads * seq_len)
    oo, oa = ob.alloc(n * width), ob.alloc(n * n_heads * seq_len)
    hip.attention(hip.upload(q), go, ga, 0, [K.Window(a, s, (x, y)) for a, s, x, y in windows], spec)
    ob.attention(ob.upload(q), oo, oa, 0, windows, n_heads, n_heads // n_kv, hs, kv_dim, seq_len)
    out_g, out_o = hip.read(go, n * width), ob.read(oo, n * width)
    assert_bits_equal(out_g, out_o, "attention out, every row")
    ga_h, oa_h = hip.read(ga, n * n_heads * seq_len), ob.read(oa, n * n_heads * seq_len)
    for r, (a, s, x, y) in enumerate(windows):
        cnt = (y - x) + s - a + 1
        for h in range(n_heads):
            base = (r * n_heads + h) * seq_len
            assert_bits_equal(ga_h[base:base + cnt], oa_h[base:base + cnt], f"att row {r} head {h}")
    hip.close()
    return out_g


@pytest.mark.parametrize("n_heads,n_kv,hs", [(8, 8, 64), (16, 8, 128), (24, 8, 64), (16, 4, 128), (16, 2, 64)])
def test_matrix_core_attention_every_row(n_heads, n_kv, hs):
    # kv_mul 1, 2, 3 (one query head per workgroup), 4 and 8; 70 rows = two
    # or more full blocks of 32 / G rows and a partial one; windows of 1101
    # to 1170 positions, i.e. across 32-position chunks with each row ending
    # in a different one
    _mx_case(1400, n_heads, n_kv, hs, [(0, 1100 + i, 0, 0) for i in range(70)], 101 + hs + n_heads)
    # a shared prefix of 300 slots, then each row's own suffix
    _mx_case(1500, n_heads, n_kv, hs, [(600, 1400 + i, 0, 300) for i in range(45)], 102 + hs + n_heads)


@pytest.mark.parametrize("n_heads,n_kv,hs", [(8, 8, 64), (16, 8, 128)])
def test_matrix_core_attention_past_4096_positions(n_heads, n_kv, hs):
    # windows of 4500-4570 positions in 32-pair blocks and a partial one
    _mx_case(4700, n_heads, n_kv, hs, [(0, 4500 + i, 0, 0) for i in range(70)], 301 + hs)


@pytest.mark.parametrize("hs", [64, 128])
def test_matrix_core_attention_ignores_v_past_a_window(hs):
    # row 0 of the first block ends at slot 1100; slot 1101 holds +inf in a
    # few dims: the rows whose windows reach it are inf there (as the
    # reference), row 0 never reads it and stays finite
    out = _mx_case(1300, 16, 4, hs, [(0, 1100 + i, 0, 0) for i in range(40)], 7 + hs, inf_slot=1101)
    width = 16 * hs
    assert np.isfinite(out[:width]).all()
    assert np.isinf(out[width:2 * width]).any()


# ---- contract checks -----------------------------------------------------------

def test_matrix_read_checks_sizes(hip):
    m = hip.synthetic_matrix("q8_0", 64, 128, 3)
    assert hip.matrix_shape(m) == ("q8_0", 64, 128)
    q, s = hip.read_matrix(m)
    assert q.shape == (64, 128) and s.shape == (64, 4)
    with pytest.raises(ValueError):
        hip.read_matrix(m, "q8_0", 128, 128)
    small = np.empty(64 * 64, np.int8)
    sc = np.empty(64 * 4, np.float32)
    rc = hip._L.kr_matrix_read(hip.ctx, m, small.ctypes.data, small.nbytes, sc.ctypes.data, sc.nbytes)
    assert rc != 0


def test_mfma_probe_refuses_runaway_sizes(hip):
    with pytest.raises(RuntimeError):
        hip.mfma_rate(0, 1 << 20, 1 << 20)
