"""Op-level parity of the HIP backend against the oracle's restatement of the
reference cpu backend: every op, bit for bit, through the C ABI.

The int8 stages (activation quants, per-block i32 dots) and every f32 output
are compared as raw bits."""

import numpy as np
import pytest

import kernrt_amd as K
import oracle as O
from helpers import assert_bits_equal, product_matrix

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    h = K.open("hip")
    yield h
    h.close()


def edge_rows(width):
    """Rows that hit the quantizer's special cases (quant.rs:856-874)."""
    rng = np.random.default_rng(7)
    rows = [rng.normal(size=width), rng.normal(size=width) * 1e-3, np.zeros(width),
            rng.uniform(-1, 1, size=width) * 300.0]
    r = np.zeros(width)
    r[0], r[1], r[2], r[3], r[4] = 127.0, 2.5, -2.5, 0.5, -0.5  # exact .5 ties at scale 1
    rows.append(r)
    r = rng.normal(size=width)
    r[5], r[40 % width] = np.nan, np.inf  # NaN ignored by amax; inf poisons its block to NaN*0
    rows.append(r)
    rows.append(np.full(width, 1e-40))  # subnormal block: d underflows, inv overflows
    rows.append(np.full(width, -3.0e38))
    return np.array(rows, dtype=np.float32)


@pytest.mark.parametrize("width", [32, 576, 960, 2560])
def test_quantize_is_bit_exact(hip, width):
    x = edge_rows(width)
    buf = hip.upload(x)
    q, s, h = hip.dbg_quantize(buf, x.shape[0], width)
    for r in range(x.shape[0]):
        wq, ws, wh = O.quantize(x[r])
        nb = width // 32
        assert np.array_equal(q[r * width:(r + 1) * width], wq), f"row {r} quants"
        assert_bits_equal(s[r * nb:(r + 1) * nb], ws, f"row {r} scales")
        assert np.array_equal(h[r * nb:(r + 1) * nb], wh), f"row {r} f16 scales"


def test_quantize_scales_across_the_f16_range(hip):
    # block maxima from 2^-64 to 2^63 (random mantissas): the f16 scale bits
    # cover zero, subnormal, normal and infinite results and their rounding
    rng = np.random.default_rng(11)
    nb = 128
    m = 127.0 * np.exp2(np.arange(nb) - 64.0) * (1.0 + rng.uniform(0.0, 1.0, size=nb))
    x = (np.repeat(m, 32) * rng.uniform(-1.0, 1.0, size=nb * 32)).astype(np.float32)
    x[::32] = m.astype(np.float32)  # each block's max is its first element
    q, s, h = hip.dbg_quantize(hip.upload(x), 1, nb * 32)
    wq, ws, wh = O.quantize(x)
    assert np.array_equal(q, wq)
    assert_bits_equal(s, ws, "scales")
    assert np.array_equal(h, wh), "f16 scales"


SHAPES = [(1536, 576), (960, 960), (320, 960), (2560, 960), (960, 2560), (36, 8192), (100, 96)]


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", SHAPES)
def test_block_dots_are_exact(hip, storage, shape):
    n, k = shape
    if storage == "q8_0x4" and n % 4:
        pytest.skip("Q8_0x4 needs out_dim % 4 == 0")
    rng = np.random.default_rng(n * 31 + k)
    m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), storage)
    x = rng.normal(size=(3, k)).astype(np.float32)
    mat = hip.upload_matrix(product_matrix(m))
    got = hip.dbg_block_dots(mat, hip.upload(x), 3, n, k)
    xq = np.concatenate([O.quantize(x[r])[0] for r in range(3)])
    assert np.array_equal(got, m.block_dots(xq))
    hip.free_matrix(mat)


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 7])
def test_matmul_matches_cpu_project(hip, storage, shape, rows):
    n, k = shape
    if storage == "q8_0x4" and n % 4:
        pytest.skip("Q8_0x4 needs out_dim % 4 == 0")
    rng = np.random.default_rng(n + 7 * k + rows)
    m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), storage)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    mat = hip.upload_matrix(product_matrix(m))
    y = hip.alloc(rows * n)
    hip.matmul(mat, hip.upload(x), y, rows)
    assert_bits_equal(hip.read(y, rows * n), m.project_cpu(x).ravel(), f"{storage} {shape} rows={rows}")
    hip.free_matrix(mat)


# Row counts that take the int8 MFMA GEMM: partial and whole 32-row tiles.
@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("rows", [8, 33, 128])
def test_gemm_matches_cpu_project(hip, storage, shape, rows):
    test_matmul_matches_cpu_project(hip, storage, shape, rows)


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", [(1536, 576), (100, 96), (36, 8192), (260, 128)])
def test_gemm_block_dots_are_exact(hip, storage, shape):
    n, k = shape
    if storage == "q8_0x4" and n % 4:
        pytest.skip("Q8_0x4 needs out_dim % 4 == 0")
    rows = 37
    rng = np.random.default_rng(n * 29 + k)
    m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), storage)
    x = (rng.normal(size=(rows, k)) * rng.uniform(0.01, 10, size=(rows, 1))).astype(np.float32)
    x[3] = 0.0
    mat = hip.upload_matrix(product_matrix(m))
    got = hip.dbg_block_dots(mat, hip.upload(x), rows, n, k)
    xq = np.concatenate([O.quantize(x[r])[0] for r in range(rows)])
    assert np.array_equal(got, m.block_dots(xq))
    hip.free_matrix(mat)


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", [(2048, 8192), (8192, 2048)])
def test_gemm_at_1p7b_shapes(hip, storage, shape):
    # SmolLM2-1.7B down and gate/up projections with a 128-token prompt
    test_matmul_matches_cpu_project(hip, storage, shape, 128)


# The chain-split form (each of the four partial sums on its own workgroups,
# the planes added by the consumer): partial and whole 64-row tiles, one
# block per partial sum (k = 128) up to 64, and the 1.7B down shape.
@pytest.mark.parametrize("shape,rows", [((960, 2560), 8), ((960, 2560), 33), ((100, 128), 64), ((36, 8192), 128),
                                        ((100, 128), 2048), ((36, 8192), 2048), ((2048, 8192), 128)])
def test_split_gemm_matches_cpu_project(hip, shape, rows):
    n, k = shape
    rng = np.random.default_rng(n + 5 * k + rows)
    m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), "q8_0")
    x = rng.normal(size=(rows, k)).astype(np.float32)
    x[rows // 2] = 0.0
    mat = hip.upload_matrix(product_matrix(m))
    y4 = hip.alloc(4 * rows * n)
    hip.matmul_split(mat, hip.upload(x), y4, rows)
    p = hip.read(y4, 4 * rows * n).reshape(4, rows * n)
    got = ((p[0] + p[1]) + p[2]) + p[3]  # float32 adds, the consumer's order (dot.rs:45)
    want = m.project_cpu(x).ravel()
    assert_bits_equal(got, want, f"split {shape} rows={rows}")
    # again on the workspace the first call left
    hip.matmul_split(mat, None, y4, rows)
    p2 = hip.read(y4, 4 * rows * n).reshape(4, rows * n)
    assert_bits_equal(p2.ravel(), p.ravel(), "split on the kept workspace")
    hip.free_matrix(mat)


def test_split_gemm_contract(hip):
    rng = np.random.default_rng(3)
    m = O.Matrix(rng.normal(0, 0.02, size=(64, 96)).astype(np.float32), "q8_0")
    mat = hip.upload_matrix(product_matrix(m))
    x = hip.upload(rng.normal(size=(8, 96)).astype(np.float32))
    with pytest.raises(RuntimeError):  # in_dim % 128 != 0: the partial sums differ in length
        hip.matmul_split(mat, x, hip.alloc(4 * 8 * 64), 8)
    m2 = O.Matrix(rng.normal(0, 0.02, size=(64, 128)).astype(np.float32), "q8_0")
    mat2 = hip.upload_matrix(product_matrix(m2))
    hip.quantize_rows(hip.upload(rng.normal(size=(8, 128)).astype(np.float32)), 8, 128)
    with pytest.raises(RuntimeError):  # the workspace holds row-major blocks
        hip.matmul_split(mat2, None, hip.alloc(4 * 8 * 64), 8)
    hip.free_matrix(mat)
    hip.free_matrix(mat2)


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
def test_classify_matches_cpu_logits(hip, storage):
    rng = np.random.default_rng(11)
    n, k = 4096, 960
    w = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
    w[17, 64:96] = 0.0  # an all-zero block
    m = O.Matrix(w, storage)
    x = rng.normal(size=k).astype(np.float32)
    mat = hip.upload_matrix(product_matrix(m))
    y = hip.alloc(n)
    hip.classify(mat, hip.upload(x), y)
    assert_bits_equal(hip.read(y, n), m.logits_cpu(x), storage)


def test_classify_requantizes_blocks_without_a_127():
    # quant.rs:232-235: x86 logits re-quantize each decoded Q8_0x4 row; a block
    # whose largest |q| is not 127 then gets new quants and scale. Such
    # blocks come only from hand-made storage, so build one from raw records.
    hip = K.open("hip")
    rng = np.random.default_rng(12)
    n, k = 64, 256
    blocks = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), "q8_0x4").q8_0x4_blocks()
    rec = blocks.reshape(-1, 136).copy()
    q = rec[:, 8:].view(np.int8)
    q[5] = (q[5].astype(np.int32) * 3 // 5).astype(np.int8)   # max |q| ~ 76 in block 5
    q[9] = np.clip(q[9], -100, 100)
    m = O.Matrix.from_q8_0x4_blocks(rec.ravel(), n, k)
    x = rng.normal(size=k).astype(np.float32)
    mat = hip.upload_matrix(K.Q8Matrix("q8_0x4", n, k, blocks=rec.ravel()))
    y = hip.alloc(n)
    hip.classify(mat, hip.upload(x), y)
    assert_bits_equal(hip.read(y, n), m.logits_cpu(x), "requantized classifier")
    hip.close()


def pair(hip, name="cpu", weights=None, **kv):
    return O.Backend(name, weights, **kv)


def test_rms_norm_and_qk_norm(hip):
    rng = np.random.default_rng(13)
    ob = O.Backend("cpu")
    for rows, dim in [(1, 960), (5, 2048), (3, 576), (2, 33), (512, 960), (256, 2048), (64, 1536)]:
        x = (rng.normal(size=rows * dim) * 3).astype(np.float32)
        w = rng.normal(size=dim).astype(np.float32)
        for eps in (1e-5, 1e-6):
            go, gx, gw = hip.alloc(rows * dim), hip.upload(x), hip.upload(w)
            oo, ox, ow = ob.alloc(rows * dim), ob.upload(x), ob.upload(w)
            hip.rms_norm(go, gx, gw, rows, dim, eps)
            ob.rms_norm(oo, ox, ow, rows, dim, eps)
            assert_bits_equal(hip.read(go, rows * dim), ob.read(oo, rows * dim), f"rms_norm {rows}x{dim}")
    for rows, width, head in [(1, 2048, 128), (4, 1024, 64), (3, 32, 8), (300, 2048, 128), (500, 960, 64),
                              (2, 99, 33), (3, 512, 256)]:
        v = rng.normal(size=rows * width).astype(np.float32)
        w = rng.normal(size=head).astype(np.float32)
        gv, ov = hip.upload(v), ob.upload(v)
        hip.qk_norm(gv, rows, width, head, hip.upload(w), 1e-6)
        ob.qk_norm(ov, rows, width, head, ob.upload(w), 1e-6)
        assert_bits_equal(hip.read(gv, rows * width), ob.read(ov, rows * width), f"qk_norm {width}/{head}")


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope(hip, interleaved):
    rng = np.random.default_rng(14)
    ob = O.Backend("cpu")
    for qw, kvw, hs, theta in [(960, 320, 64, 1e5), (2048, 1024, 128, 1e6), (32, 16, 8, 1e4)]:
        rows = 6
        positions = [0, 1, 511, 767, 2047, 8191]
        q = rng.normal(size=rows * qw).astype(np.float32)
        k = rng.normal(size=rows * kvw).astype(np.float32)
        gq, gk, oq, okb = hip.upload(q), hip.upload(k), ob.upload(q), ob.upload(k)
        hip.rope(gq, gk, qw, kvw, rows, positions, K.RopeSpec(hs, theta, interleaved))
        ob.rope(oq, okb, qw, kvw, rows, positions, hs, theta, interleaved)
        assert_bits_equal(hip.read(gq, rows * qw), ob.read(oq, rows * qw), f"rope q {qw}")
        assert_bits_equal(hip.read(gk, rows * kvw), ob.read(okb, rows * kvw), f"rope k {kvw}")


def _attention_case(seq_len, n_heads, n_kv, hs, windows, seed):
    rng = np.random.default_rng(seed)
    emb = O.Matrix(rng.normal(0, 0.02, size=(8, 32)).astype(np.float32), "q8_0")
    ow = O.Weights(1)
    ow.set_embedding(emb)
    kv_dim = n_kv * hs
    hip = K.open("hip")
    hip.bind_handles(hip.upload_matrix(product_matrix(emb)), 0xFFFFFFFF, [{}])
    hip.prepare(None, K.KvSpec(1, kv_dim, seq_len))
    ob = O.Backend("cpu", ow, n_layers=1, kv_dim=kv_dim, seq_len=seq_len)
    # fill the cache on both sides through kv_write
    slots = np.arange(seq_len)
    kk = rng.normal(size=seq_len * kv_dim).astype(np.float32)
    vv = rng.normal(size=seq_len * kv_dim).astype(np.float32)
    hip.kv_write(0, slots, hip.upload(kk), hip.upload(vv), seq_len)
    ob.kv_write(0, slots, ob.upload(kk), ob.upload(vv), seq_len)
    n = len(windows)
    width = n_heads * hs
    q = (rng.normal(size=n * width) * 2).astype(np.float32)
    spec = K.AttnSpec(n_heads, n_heads // n_kv, hs, kv_dim, seq_len)
    go, ga = hip.alloc(n * width), hip.alloc(n * n_heads * seq_len)
    oo, oa = ob.alloc(n * width), ob.alloc(n * n_heads * seq_len)
    hip.attention(hip.upload(q), go, ga, 0, [K.Window(a, s, (x, y)) for a, s, x, y in windows], spec)
    ob.attention(ob.upload(q), oo, oa, 0, windows, n_heads, n_heads // n_kv, hs, kv_dim, seq_len)
    assert_bits_equal(hip.read(go, n * width), ob.read(oo, n * width), "attention out")
    # the probabilities left in `att`
    ga_h, oa_h = hip.read(ga, n * n_heads * seq_len), ob.read(oa, n * n_heads * seq_len)
    for r, (a, s, x, y) in enumerate(windows):
        cnt = (y - x) + s - a + 1
        for h in range(n_heads):
            base = (r * n_heads + h) * seq_len
            assert_bits_equal(ga_h[base:base + cnt], oa_h[base:base + cnt], f"att row {r} head {h}")
    hip.close()


def test_attention_decode_windows():
    _attention_case(1024, 15, 5, 64, [(0, 0, 0, 0), (0, 511, 0, 0), (0, 767, 0, 0)], 15)


@pytest.mark.parametrize("n_heads,n_kv,hs", [(32, 32, 64), (16, 8, 128), (16, 1, 64), (12, 1, 32), (24, 8, 64)])
def test_attention_head_groupings(n_heads, n_kv, hs):
    # kv_mul 1 (1.7B), 2 (Qwen3), 16 and 12 (multi-query), 3 (LFM2)
    _attention_case(600, n_heads, n_kv, hs, [(0, 599, 0, 0), (0, 37, 0, 0), (10, 300, 0, 5)], n_heads + hs)


def test_attention_shared_and_multi_windows():
    # prefill_shared / prefill_multi windows (llama.rs:552-647)
    _attention_case(64, 4, 2, 8, [(0, 2, 0, 0), (3, 4, 0, 3), (5, 8, 0, 3), (9, 9, 0, 3), (10, 20, 0, 0)], 16)


@pytest.mark.parametrize("n_heads,n_kv,hs", [(4, 4, 64), (8, 4, 128), (6, 2, 64), (16, 2, 32), (8, 1, 128)])
def test_attention_prefill_rows(n_heads, n_kv, hs):
    # prefill windows (row i attends to slots 0..=i, or a shared prefix plus
    # its own suffix): blocks of rows that share one window layout, 70 rows =
    # several blocks and a partial one, windows across 64-position tiles
    _attention_case(160, n_heads, n_kv, hs, [(0, i, 0, 0) for i in range(70)], 40 + hs)
    _attention_case(160, n_heads, n_kv, hs, [(90, 90 + i, 3, 71) for i in range(45)], 41 + hs)


@pytest.mark.parametrize("n_heads,n_kv,hs", [(8, 8, 64), (6, 2, 64), (16, 2, 32), (8, 4, 128)])
def test_attention_prefill_rows_many_tiles(n_heads, n_kv, hs):
    # windows of 301 to 340 positions: six K and six V tiles per block, so the
    # tiles pass through both register sets several times; kv_mul 3 leaves a
    # block with an odd number of (row, head) pairs
    _attention_case(400, n_heads, n_kv, hs, [(0, 300 + i, 0, 0) for i in range(40)], 42 + hs + n_heads)


def test_attention_prefill_rows_1p7b_shape():
    # the 128-row prefill of the 1.7B shape: 32 heads, kv_mul 1, head_dim 64
    _attention_case(160, 32, 32, 64, [(0, i, 0, 0) for i in range(128)], 43)


def test_attention_long_context_uses_global_scores():
    # more scores than fit in LDS: the kernel keeps them in `att`
    _attention_case(16384, 2, 1, 128, [(0, 13000, 0, 0), (100, 16383, 0, 0)], 17)


def test_elementwise_ops(hip):
    rng = np.random.default_rng(18)
    ob = O.Backend("cpu")
    n = 4099
    a = (rng.normal(size=n) * 4).astype(np.float32)
    b = rng.normal(size=n).astype(np.float32)
    a[:4] = [0.0, -0.0, 88.5, -104.0]
    ga, gb, oa, obb = hip.upload(a), hip.upload(b), ob.upload(a), ob.upload(b)
    hip.silu_mul(ga, gb, n)
    ob.silu_mul(oa, obb, n)
    assert_bits_equal(hip.read(ga, n), ob.read(oa, n), "silu_mul")
    hip.add_in_place(ga, gb, n)
    ob.add_in_place(oa, obb, n)
    assert_bits_equal(hip.read(ga, n), ob.read(oa, n), "add_in_place")
    # mul over slices of one buffer (the LFM2 B*x pattern), and an overlapping case
    x = rng.normal(size=3 * 100).astype(np.float32)
    for (oo, ao, bo, ln) in [(0, 0, 200, 100), (5, 0, 200, 100), (0, 5, 7, 150), (0, 0, 0, 300)]:
        gx, ox = hip.upload(x), ob.upload(x)
        hip.mul(gx, oo, gx, ao, gx, bo, min(ln, 300 - max(oo, ao, bo)))
        ob.mul(ox, oo, ox, ao, ox, bo, min(ln, 300 - max(oo, ao, bo)))
        assert_bits_equal(hip.read(gx, 300), ob.read(ox, 300), f"mul {oo},{ao},{bo}")
    # copy with overlap has memmove semantics (cpu.rs:230-232)
    for (so, do, ln) in [(0, 10, 100), (10, 0, 100), (0, 200, 100)]:
        gx, ox = hip.upload(x), ob.upload(x)
        hip.copy(gx, so, gx, do, ln)
        ob.copy(ox, so, ox, do, ln)
        assert_bits_equal(hip.read(gx, 300), ob.read(ox, 300), f"copy {so}->{do}")


def test_conv_prefill_and_decode(hip):
    rng = np.random.default_rng(19)
    ob = O.Backend("cpu")
    dim, k, rows = 1536, 3, 9
    h = rng.normal(size=rows * dim).astype(np.float32)
    kw = rng.normal(size=dim * k).astype(np.float32)
    go, oo = hip.alloc(rows * dim), ob.alloc(rows * dim)
    hip.conv_prefill(go, hip.upload(h), hip.upload(kw), rows, dim, k)
    ob.conv_prefill(oo, ob.upload(h), ob.upload(kw), rows, dim, k)
    assert_bits_equal(hip.read(go, rows * dim), ob.read(oo, rows * dim), "conv_prefill")
    st0 = rng.normal(size=(k - 1) * dim).astype(np.float32)
    gs, os_ = hip.upload(st0), ob.upload(st0)
    gk, okk = hip.upload(kw), ob.upload(kw)
    for r in range(4):
        xr = h[r * dim:(r + 1) * dim]
        gx, ox = hip.upload(xr), ob.upload(xr)
        go1, oo1 = hip.alloc(dim), ob.alloc(dim)
        hip.conv_decode(go1, gx, gk, gs, dim, k)
        ob.conv_decode(oo1, ox, okk, os_, dim, k)
        assert_bits_equal(hip.read(go1, dim), ob.read(oo1, dim), f"conv_decode out {r}")
        assert_bits_equal(hip.read(gs, (k - 1) * dim), ob.read(os_, (k - 1) * dim), f"conv_decode ring {r}")


def test_argmax_tie_rule(hip):
    v = np.array([1.0, 3.0, 3.0, 2.0, -0.0, 0.0], np.float32)
    for arr, want in [(v, 2), (np.array([0.0, -0.0], np.float32), 0), (np.array([-0.0, 0.0, -0.0], np.float32), 1)]:
        b = hip.upload(arr)
        hip.argmax(b, arr.size, 0)
        assert int(hip.read_tokens(1)[0]) == want == O.argmax(arr)
    rng = np.random.default_rng(20)
    big = rng.normal(size=151936).astype(np.float32)
    big[[5, 100000, 150000]] = 9.0
    b = hip.upload(big)
    hip.argmax(b, big.size, 3)
    assert int(hip.read_tokens(4)[3]) == O.argmax(big) == 150000


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("shape", [(96, 960), (2560, 960), (2048, 8192)])
def test_synthetic_weights_quantize_as_the_oracle(hip, storage, shape):
    # the benchmarks' device-generated weights (kr_matrix_synthetic): the
    # stored bytes equal the reference quantization (quant.rs:544-557,
    # 124-164) of the very f32 values the generator drew
    n, k = shape
    mat = hip.synthetic_matrix(storage, n, k, 41)
    vals = hip.synthetic_values(n * k, 41, 0.02).reshape(n, k)
    om = O.Matrix(vals, storage)
    q, s = hip.read_matrix(mat, storage, n, k)
    if storage == "q8_0":
        oq, os_ = om.q8_0_data()
        assert np.array_equal(q.ravel(), oq) and np.array_equal(s.ravel().view(np.uint32), os_.view(np.uint32))
    else:
        assert np.array_equal(K.backends.q8_0x4_records(q, s), om.q8_0x4_blocks())
    hip.free_matrix(mat)
