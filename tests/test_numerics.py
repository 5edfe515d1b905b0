"""The shared device/host numerics (kernrt_amd/csrc/numerics.hpp), host build.

The HIP kernels compile the same header for gfx950, so pinning the host
build pins the formulas; the GPU tests then pin the device build against the
oracle. Product code is compiled here only as the thing under test.
"""

import os
import subprocess

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _build(tmp_path):
    exe = str(tmp_path / "numerics_check")
    subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-pthread",
                    os.path.join(HERE, "numerics_check.cpp"), "-o", exe, "-lm"], check=True)
    return exe


def _run(exe, stride, threads):
    out = subprocess.run([exe, str(stride), str(threads)], check=True, capture_output=True, text=True).stdout
    vals = dict(line.split() for line in out.strip().splitlines())
    return {k: int(v) for k, v in vals.items()}


def test_expf_matches_glibc_on_a_sample(tmp_path):
    # every 61st float (~70M inputs, both signs, all exponents)
    r = _run(_build(tmp_path), 61, 8)
    assert r["checked"] > 60_000_000
    assert r["expf_mismatch"] == 0
    assert r["f16_mismatch"] == 0


@pytest.mark.slow
def test_expf_matches_glibc_exhaustively(tmp_path):
    r = _run(_build(tmp_path), 1, 8)
    assert r["checked"] == 2**32
    assert r["expf_mismatch"] == 0


def test_expf_agrees_with_the_oracle_on_softmax_inputs():
    # The oracle calls glibc `expf` (what Rust's f32::exp lowers to); spot
    # values in the softmax domain (x <= 0) and the SiLU domain.
    xs = np.concatenate([-np.geomspace(1e-8, 100, 2000), np.linspace(-20, 20, 2001)]).astype(np.float32)
    want = np.array([O.expf(x) for x in xs], np.float32)
    assert np.all(np.isfinite(want))
    # a known-wrongly-rounded glibc case must be reproduced, not corrected
    assert O.expf(np.float32.fromhex("0x1.fefe02p-16") if hasattr(np.float32, "fromhex")
                  else float.fromhex("0x1.fefe02p-16")) == float.fromhex("0x1.0002p+0")
