"""The kernels' parallel form of the reference's serial f32 sums (the RMS sum
of squares, cpu.rs:635-641; the softmax sum, cpu.rs:575-630): s = +0, then
s += v[i] in order, each add rounded. The GPU result must be the sequential
f32 sum bit for bit whenever the parallel form reports that it applied, and
it must apply to the ordinary inputs the model produces (squares and
exponentials); where it does not apply the kernels run the serial chain,
checked here too.

Inputs: squares of normal values over 60 binades of scale, exponentials,
small integers and dyadic values (exact ties in the sum's grid), powers of
two, zeros (leading and scattered), subnormals, and non-finite values (which
must leave the parallel form and go to the chain)."""

import numpy as np
import pytest

import kernrt_amd as K

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 5, 63, 64, 65, 127, 515, 960, 1024, 1025, 1536, 2048]


@pytest.fixture(scope="module")
def hip():
    h = K.open("hip")
    yield h
    h.close()


def _serial(v):
    """The reference's loop: f32 adds in order from +0."""
    out = np.empty(v.shape[0], np.float32)
    with np.errstate(over="ignore"):
        acc = np.add.accumulate(v.astype(np.float32), axis=1, dtype=np.float32)
    out[:] = acc[:, -1]
    # np.add.accumulate starts from v[0] rather than +0 + v[0]: the same bits
    # for non-negative terms (+0 + x = x), so no adjustment is needed
    return out


def _vectors(kind, n, count, rng):
    if kind == "squares":
        scale = np.ldexp(1.0, rng.integers(-30, 30, size=(count, 1))).astype(np.float32)
        x = rng.normal(size=(count, n)).astype(np.float32) * scale
        return x * x
    if kind == "exps":
        return np.exp(rng.normal(size=(count, n)) * 3.0 - 4.0).astype(np.float32)
    if kind == "small_ints":
        return rng.integers(0, 16, size=(count, n)).astype(np.float32)
    if kind == "dyadic":
        return np.ldexp(rng.integers(0, 1024, size=(count, n)), rng.integers(-20, -12, size=(count, n))).astype(np.float32)
    if kind == "powers":
        v = np.ldexp(1.0, rng.integers(-15, 15, size=(count, n))).astype(np.float32)
        v[:, :10] = 0.0
        return v
    if kind == "zeros":
        x = rng.normal(size=(count, n)).astype(np.float32)
        v = x * x
        v[rng.random(size=(count, n)) < 0.2] = 0.0
        v[: count // 2, : n // 3] = 0.0
        return v
    if kind == "subnormal":
        return rng.integers(0, 1 << 23, size=(count, n), dtype=np.uint32).view(np.float32)
    raise ValueError(kind)


KINDS = ["squares", "exps", "small_ints", "dyadic", "powers", "zeros", "subnormal"]


@pytest.mark.parametrize("waves", [1, 2, 4, 16])
@pytest.mark.parametrize("kind", KINDS)
def test_parallel_serial_sum_matches_the_loop(hip, kind, waves):
    rng = np.random.default_rng(7 + KINDS.index(kind))
    for n in SIZES:
        v = _vectors(kind, n, 256, rng)
        want = _serial(v)
        fast, applied, chain, _, _ = hip.dbg_serial_sum(v, waves)
        assert np.array_equal(chain.view(np.uint32), want.view(np.uint32)), f"{kind} n={n}: the chain"
        bad = applied & (fast.view(np.uint32) != want.view(np.uint32))
        assert not bad.any(), f"{kind} n={n}: {int(bad.sum())} parallel sums differ"
        if kind in ("squares", "exps") and n >= 64:
            # the model's inputs: the parallel form must be the one that runs
            assert applied.mean() > 0.99, f"{kind} n={n}: applied to {applied.mean():.3f}"


@pytest.mark.parametrize("waves", [1, 2, 4, 16])
def test_parallel_serial_sum_leaves_non_finite_input_to_the_chain(hip, waves):
    rng = np.random.default_rng(3)
    for n in (64, 960, 2048):
        v = _vectors("squares", n, 8, rng)
        v[0, n // 2] = np.inf
        v[1, 0] = np.nan
        v[2, n - 1] = np.inf
        v[3, :] = np.float32(3e38)  # the sum overflows
        fast, applied, chain, _, _ = hip.dbg_serial_sum(v, waves)
        assert not applied[:4].any()
        want = _serial(v)
        same = (chain.view(np.uint32) == want.view(np.uint32)) | (np.isnan(chain) & np.isnan(want))
        assert same.all()
        assert applied[4:].all()
        assert np.array_equal(fast[4:].view(np.uint32), want[4:].view(np.uint32))
