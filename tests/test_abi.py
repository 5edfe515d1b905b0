"""The C ABI boundary, without a GPU: the library loads, exports every entry
point include/*.h declares, and reports a missing device the way
`BackendError::detail` does (src/backends/mod.rs:190-213)."""

import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kernrt_hip.h", "kernrt_llm.h")]


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(krl?_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_trait_surface():
    names = declared_symbols()
    # one entry per `Backend` method (mod.rs:264-404)
    for op in ["open", "name", "storage", "prepare", "alloc", "upload", "read", "embed", "copy", "rms_norm",
               "qk_norm", "rope", "project", "project_qkv", "project_gate_up", "kv_write", "attention",
               "add_in_place", "mul", "conv_prefill", "conv_decode", "silu_mul", "logits"]:
        assert f"kr_{op}" in names, op


def test_library_exports_every_declared_symbol():
    from kernrt_amd import _lib
    lib = _lib.load()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.EXPORTED) == declared_symbols()


def test_open_without_a_device_is_a_detailed_backend_error():
    import torch  # noqa: F401  (only to learn whether this host has a GPU)
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the gpu tests")
    import kernrt_amd
    with pytest.raises(kernrt_amd.BackendError) as e:
        kernrt_amd.open("hip")
    assert e.value.requested == "hip"
    assert e.value.detail is not None and "no HIP device" in e.value.detail
    assert "is unavailable" in str(e.value)


def test_unknown_backend_is_an_error():
    # tests/backends.rs:196-204: `open("cuda")` must fail, naming what exists
    import kernrt_amd
    with pytest.raises(kernrt_amd.BackendError) as e:
        kernrt_amd.open("cuda")
    assert e.value.requested == "cuda" and e.value.detail is None
    assert "available" in str(e.value) and "hip" in str(e.value)
    assert kernrt_amd.available() == ["hip"]


def test_q8_0x4_records_invert_the_upload_deinterleave():
    # the host repack that turns the device layout (row-major int8 + f16 scale
    # bits) back into the reference's 136-byte records (quant.rs:113-164)
    import numpy as np
    import kernrt_amd as K
    import oracle as O
    rng = np.random.default_rng(4)
    n, k = 64, 96
    m = O.Matrix(rng.normal(0, 0.02, size=(n, k)).astype(np.float32), "q8_0x4")
    rec = m.q8_0x4_blocks().reshape(n // 4, k // 32, 136)
    q, s = m.to_row_major()  # int8 [n*k] and the widened f32 scales
    bits = rec[:, :, :8].copy().view(np.uint16).reshape(n // 4, k // 32, 4).transpose(0, 2, 1).reshape(n, k // 32)
    assert np.array_equal(np.array([O.f16_scale_to_f32(int(b)) for b in bits.ravel()], np.float32), s)
    got = K.backends.q8_0x4_records(q.reshape(n, k), bits)
    assert np.array_equal(got, rec.ravel())
