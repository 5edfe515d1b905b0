"""Reader for the `safetensors` format, as the reference reads it
(src/formats/safetensors.rs).

Layout: a little-endian u64 header length, that many bytes of UTF-8 JSON, then
the data. The JSON maps tensor names to ``{"dtype", "shape", "data_offsets":
[start, end]}`` (byte ranges into the data), plus an optional
``"__metadata__"`` entry that is not a tensor. Only F32, BF16 and F16 are read.
The file is untrusted: every offset and shape is checked against the file size
before it is used (safetensors.rs:176-262).

The file is memory-mapped; `load_raw` keeps bf16 payloads as their bit
patterns (safetensors.rs:170-173, 319-361) so a bf16 checkpoint reaches the
device without a pass through f32 on the host.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Callable, Dict, Tuple, Union

import numpy as np


class SafeTensorsError(Exception):
    """Everything that can go wrong reading a safetensors file
    (safetensors.rs:30-96)."""


class HeaderTooShort(SafeTensorsError):
    def __init__(self, file_len: int, needed: int):
        super().__init__(f"need {needed} bytes for the header, the file holds {file_len}")
        self.file_len, self.needed = file_len, needed


class InvalidJson(SafeTensorsError):
    def __init__(self, err: Exception):
        super().__init__(f"the header is not UTF-8 JSON ({err})")


class InvalidHeader(SafeTensorsError):
    def __init__(self, msg: str):
        super().__init__(f"malformed header: {msg}")


class UnsupportedDtype(SafeTensorsError):
    def __init__(self, dtype: str):
        super().__init__(f"dtype {dtype!r} cannot be read; F32, BF16 and F16 can")
        self.dtype = dtype


class InvalidOffsets(SafeTensorsError):
    def __init__(self, name: str, start: int, end: int):
        super().__init__(f"bytes [{start}, {end}) of {name!r} disagree with its dtype, its shape or the file length")
        self.name, self.start, self.end = name, start, end


_WIDTH = {"F32": 4, "BF16": 2, "F16": 2}


@dataclass
class RawTensor:
    """A tensor as the file stores it (safetensors.rs:307-330): dtype "F32"
    (f32 values), "BF16" (uint16 bit patterns) or "F16" (already widened to
    f32, as the reference does: nothing consumes f16 raw)."""
    dtype: str
    shape: Tuple[int, ...]
    data: np.ndarray  # flat: float32 for F32/F16, uint16 for BF16

    def widen(self) -> np.ndarray:
        """f32 values in `shape` (hf.rs:93-103): bf16 is the top half of an f32."""
        if self.dtype == "BF16":
            return (self.data.astype(np.uint32) << 16).view(np.float32).reshape(self.shape)
        return np.asarray(self.data, np.float32).reshape(self.shape)


def _as_uint(v) -> Union[int, None]:
    # serde_json's as_u64: a non-negative integer (not a bool, not a float)
    if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v >= 1 << 64:
        return None
    return v


def _decode_raw(dtype: str, raw: np.ndarray, shape: Tuple[int, ...]) -> RawTensor:
    if dtype == "F32":
        return RawTensor("F32", shape, raw.view("<f4"))
    if dtype == "BF16":
        return RawTensor("BF16", shape, raw.view("<u2"))
    # IEEE binary16 -> binary32 is exact (safetensors.rs:363-386)
    return RawTensor("F16", shape, raw.view("<f2").astype(np.float32))


def _read_with(buf: np.ndarray, decode: Callable[[str, np.ndarray, Tuple[int, ...]], object]) -> Dict[str, object]:
    """The shared, validating parser (safetensors.rs:176-262); `buf` is the
    whole file as uint8."""
    n = int(buf.size)
    if n < 8:
        raise HeaderTooShort(n, 8)
    header_len = int(buf[:8].view("<u8")[0])
    if header_len > n - 8:
        raise HeaderTooShort(n, 8 + header_len)
    try:
        header = json.loads(bytes(buf[8:8 + header_len]).decode("utf-8"))
    except (UnicodeDecodeError, ValueError) as e:
        raise InvalidJson(e) from None
    data = buf[8 + header_len:]
    if not isinstance(header, dict):
        raise InvalidHeader("the header must be a JSON object")
    out = {}
    for name, spec in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(spec, dict):
            raise InvalidHeader(f"entry {name!r} must be a JSON object")
        dtype = spec.get("dtype")
        if not isinstance(dtype, str):
            raise InvalidHeader(f"entry {name!r} lacks a string dtype")
        if dtype not in _WIDTH:
            raise UnsupportedDtype(dtype)
        shape = spec.get("shape")
        if not isinstance(shape, list):
            raise InvalidHeader(f"entry {name!r} lacks a shape list")
        dims = [_as_uint(d) for d in shape]
        if any(d is None for d in dims):
            raise InvalidHeader(f"entry {name!r}: each dimension must be a non-negative integer")
        offs = spec.get("data_offsets")
        if not isinstance(offs, list):
            raise InvalidHeader(f"entry {name!r} lacks a data_offsets list")
        start = _as_uint(offs[0]) if len(offs) > 0 else None
        end = _as_uint(offs[1]) if len(offs) > 1 else None
        if start is None or end is None:
            raise InvalidHeader(f"entry {name!r}: data_offsets must be a start and an end, non-negative integers")
        numel = 1
        for d in dims:
            numel *= d
        expected = numel * _WIDTH[dtype]
        if start > end or end > data.size or end - start != expected or expected >= 1 << 64:
            raise InvalidOffsets(name, start, end)
        out[name] = decode(dtype, data[start:end], tuple(dims))
    return out


def _map(path) -> np.ndarray:
    # an empty file cannot be mapped; read it (safetensors.rs:117-127)
    if os.path.getsize(path) == 0:
        return np.zeros(0, np.uint8)
    return np.memmap(path, dtype=np.uint8, mode="r")


def read_raw_from(buf) -> Dict[str, RawTensor]:
    """Parse a complete byte image, keeping bf16 bit patterns
    (safetensors.rs:170-173)."""
    return _read_with(np.frombuffer(buf, np.uint8) if isinstance(buf, (bytes, bytearray)) else buf, _decode_raw)


def read_from(buf) -> Dict[str, np.ndarray]:
    """Parse a complete byte image, every tensor widened to f32
    (safetensors.rs:146-168)."""
    return {k: v.widen() for k, v in read_raw_from(buf).items()}


def load_raw(path) -> Dict[str, RawTensor]:
    """Map a safetensors file and parse it without widening
    (safetensors.rs:130-136)."""
    return read_raw_from(_map(path))


def load(path) -> Dict[str, np.ndarray]:
    """Every tensor of a safetensors file, widened to f32 (safetensors.rs:117-127)."""
    return read_from(_map(path))
