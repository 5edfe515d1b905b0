"""Committed golden fixtures (tests/golden/): the reference's known answers,
and Q8 vectors the oracle wrote on fixed inputs. The CPU tests pin the
oracle to them; the GPU test holds the HIP kernels to the same bytes."""

import json
import os

import numpy as np
import pytest

import oracle as O
from helpers import assert_bits_equal

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = [("cfg1_slice", "q8_0"), ("x4_4x64", "q8_0x4"), ("x4_8x128", "q8_0x4")]


@pytest.fixture(scope="module")
def vec():
    return np.load(os.path.join(GOLD, "q8_vectors.npz"))


def test_known_answers():
    kat = json.load(open(os.path.join(GOLD, "known_answers.json")))
    vals = np.array(kat["q8_step_multiples"]["values"], np.float32)
    q, s, _ = O.quantize(vals)
    assert np.all(s == np.float32(kat["q8_step_multiples"]["scale"]))
    assert np.array_equal(q.astype(np.float32) * np.repeat(s, 32), vals)
    sm = kat["softmax_1_2_3"]
    assert np.allclose(O.softmax(sm["input"]), sm["want"], atol=sm["tol"], rtol=0)
    g = kat["gemv_hand"]
    assert list(O.Matrix(np.array(g["w"], np.float32), "f32").gemv(np.array(g["x"], np.float32))) == g["want"]


@pytest.mark.parametrize("name,storage", CASES)
def test_oracle_reproduces_the_fixtures(vec, name, storage):
    w, x = vec[f"{name}.w"], vec[f"{name}.x"]
    m = O.Matrix(w, storage)
    for r in range(x.shape[0]):
        q, s, h = O.quantize(x[r])
        assert np.array_equal(q, vec[f"{name}.xq"][r])
        assert_bits_equal(s, vec[f"{name}.xs"][r], "xs")
        assert np.array_equal(h, vec[f"{name}.xh"][r])
    if storage == "q8_0":
        q, s = m.q8_0_data()
        assert np.array_equal(q, vec[f"{name}.wq"]) and np.array_equal(s, vec[f"{name}.ws"])
    else:
        assert np.array_equal(m.q8_0x4_blocks(), vec[f"{name}.blocks"])
    assert np.array_equal(m.block_dots(vec[f"{name}.xq"].ravel()), vec[f"{name}.dots"])
    assert_bits_equal(m.project_cpu(x), vec[f"{name}.y"], "y")
    assert_bits_equal(m.logits_cpu(x[0]), vec[f"{name}.logits"], "logits")


@pytest.mark.gpu
@pytest.mark.parametrize("name,storage", CASES)
def test_hip_reproduces_the_fixtures(vec, name, storage):
    import kernrt_amd as K
    hip = K.open("hip")
    w, x = vec[f"{name}.w"], vec[f"{name}.x"]
    n, k = w.shape
    rows = x.shape[0]
    if storage == "q8_0":
        mat = hip.upload_matrix(K.Q8Matrix("q8_0", n, k, quants=vec[f"{name}.wq"], scales=vec[f"{name}.ws"]))
    else:
        mat = hip.upload_matrix(K.Q8Matrix("q8_0x4", n, k, blocks=vec[f"{name}.blocks"]))
    xb = hip.upload(x)
    q, s, h = hip.dbg_quantize(xb, rows, k)
    assert np.array_equal(q, vec[f"{name}.xq"].ravel())
    assert_bits_equal(s, vec[f"{name}.xs"].ravel(), "xs")
    assert np.array_equal(h, vec[f"{name}.xh"].ravel())
    assert np.array_equal(hip.dbg_block_dots(mat, xb, rows, n, k), vec[f"{name}.dots"])
    y = hip.alloc(rows * n)
    hip.matmul(mat, xb, y, rows)
    assert_bits_equal(hip.read(y, rows * n), vec[f"{name}.y"].ravel(), "y")
    x0 = hip.upload(x[0])
    hip.classify(mat, x0, y)
    assert_bits_equal(hip.read(y, n), vec[f"{name}.logits"], "logits")
    hip.close()
