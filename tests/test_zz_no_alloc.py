"""kr_matmul_noalloc, the entry point that allocates nothing: same bits as
kr_matmul on two calls in a row (the second with a smaller input, so it runs
over what the first left in the shared device array), for both storages and
for the GEMV (rows <= 4) and MFMA GEMM kernels; sizes past the array's limit
are refused before anything runs."""

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


def one_call(hip, mat, n, k, rows, seed):
    x = np.random.default_rng(seed).normal(size=(rows, k)).astype(np.float32)
    xb = hip.upload(x)
    y_ref, y_new = hip.alloc(rows * n), hip.alloc(rows * n)
    hip.matmul(mat, xb, y_ref, rows)
    hip.matmul_noalloc(mat, xb, y_new, rows)
    return hip.read(y_new, rows * n), hip.read(y_ref, rows * n)


@pytest.mark.parametrize("storage", ["q8_0", "q8_0x4"])
@pytest.mark.parametrize("first,second", [((160, 2048), (3, 960)), ((4, 960), (1, 576)),
                                          ((2048, 2048), (64, 1024))])
def test_noalloc_matches_matmul_twice(hip, storage, first, second):
    mats = []
    for i, (rows, k) in enumerate([first, second]):
        n = 4 * (50 + 37 * i + k // 64)
        rng = np.random.default_rng(rows * 13 + k + i)
        m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), storage)
        mat = hip.upload_matrix(product_matrix(m))
        mats.append(mat)
        got, want = one_call(hip, mat, n, k, rows, seed=i + rows)
        assert_bits_equal(got, want, f"call {i + 1}: {storage} rows={rows} k={k}")
        if i == 1:  # the oracle too, on a few rows
            x = np.random.default_rng(i + rows).normal(size=(rows, k)).astype(np.float32)
            assert_bits_equal(got.reshape(rows, n)[:2], m.project_cpu(x[:2]), "vs oracle")
    for mat in mats:
        hip.free_matrix(mat)


def test_noalloc_refuses_sizes_past_its_array(hip):
    limit = hip.matmul_noalloc_max_elems()
    assert limit == 4 << 20
    k = 1024
    rows = limit // k + 1
    m = O.Matrix(np.zeros((8, k), np.float32), "q8_0")
    mat = hip.upload_matrix(product_matrix(m))
    xb, yb = hip.alloc(rows * k), hip.alloc(rows * 8)
    with pytest.raises(RuntimeError, match="no-allocation limit"):
        hip.matmul_noalloc(mat, xb, yb, rows)
    hip.matmul_noalloc(mat, xb, yb, rows - 1)  # exactly at the limit: accepted
    assert np.all(hip.read(yb, (rows - 1) * 8) == 0)
    hip.free_matrix(mat)
