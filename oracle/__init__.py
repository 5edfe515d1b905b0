"""TEST INFRASTRUCTURE ONLY: ctypes binding of the parity oracle.

The oracle (oracle/oracle.cpp) restates the reference KernRT CPU arithmetic
for the Q8_0 / Q8_0x4 path in C++. Only tests/, ``__graft_entry__.smoke()``
and bench.py's ``cpu_baseline`` leg import this module, and only as the
checker or the timed CPU baseline; the product (``kernrt_amd``) never does.

Model builders here mirror the reference's own test fixtures:
``backends_config``/``backends_weights`` follow tests/backends.rs:24-109 and
``lfm2_weights`` follows src/arch/llm/lfm2.rs:660-766.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KERNRT_ORACLE_VARIANT=o3 loads the -O3 build of the same source (bench.py's
# second CPU figure); the default is the -O2 build.
VARIANT = os.environ.get("KERNRT_ORACLE_VARIANT", "")
LIB_PATH = os.path.join(HERE, "_build", "liboracle_o3.so" if VARIANT == "o3" else "liboracle.so")
LIB_PATHS = (os.path.join(HERE, "_build", "liboracle.so"), os.path.join(HERE, "_build", "liboracle_o3.so"))

KIND = {"f32": 0, "bf16": 1, "q8_0": 2, "q8_0x4": 3}
KIND_NAME = {v: k for k, v in KIND.items()}
PROJ = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "down": 5, "up": 6, "conv_in": 7, "conv_out": 8}

_lib = None


SOURCES = ("oracle.cpp", "capi.cpp", "oracle.hpp", "Makefile")


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (g++, -O2 -ffp-contract=off)."""
    stale = any(not os.path.exists(p) or any(os.path.getmtime(os.path.join(HERE, s)) > os.path.getmtime(p)
                                             for s in SOURCES) for p in LIB_PATHS)
    if force or stale:
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", HERE], check=True)
    return LIB_PATH


class OracleConfig(C.Structure):
    _fields_ = [
        ("dim", C.c_size_t), ("hidden_dim", C.c_size_t), ("n_layers", C.c_size_t),
        ("n_heads", C.c_size_t), ("n_kv_heads", C.c_size_t), ("vocab_size", C.c_size_t),
        ("seq_len", C.c_size_t), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("rope_interleaved", C.c_int), ("head_dim", C.c_size_t),
    ]


class OracleWindow(C.Structure):
    _fields_ = [("att_start", C.c_size_t), ("slot", C.c_size_t),
                ("shared_start", C.c_size_t), ("shared_end", C.c_size_t)]


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(LIB_PATH)
        vp, sz, f32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float)
        L.or_last_error.restype = C.c_char_p
        L.or_f32_to_f16_bits.restype = C.c_uint16
        L.or_f32_to_f16_bits.argtypes = [C.c_float]
        L.or_f16_scale_to_f32.restype = C.c_float
        L.or_f16_scale_to_f32.argtypes = [C.c_uint16]
        L.or_expf.restype = C.c_float
        L.or_expf.argtypes = [C.c_float]
        L.or_dot_q8_0_scalar.restype = C.c_float
        L.or_dot_q8_0_scalar.argtypes = [vp, vp, vp, vp, sz]
        L.or_dot_scalar.restype = C.c_float
        L.or_dot_scalar.argtypes = [vp, vp, sz]
        L.or_argmax.restype = sz
        L.or_argmax.argtypes = [vp, sz]
        L.or_lcg_fill.argtypes = [sz, C.c_uint64, vp]
        L.or_quantize.argtypes = [vp, sz, vp, vp, vp]
        L.or_softmax.argtypes = [vp, sz]
        L.or_matrix_from_f32.argtypes = [vp, sz, sz, C.c_int, C.POINTER(vp)]
        L.or_matrix_free.argtypes = [vp]
        L.or_matrix_from_q8_0.argtypes = [vp, vp, sz, sz, C.POINTER(vp)]
        L.or_matrix_from_q8_0x4_blocks.argtypes = [vp, sz, sz, C.POINTER(vp)]
        L.or_matrix_info.argtypes = [vp, C.POINTER(C.c_int), C.POINTER(sz), C.POINTER(sz)]
        L.or_matrix_decode_row.argtypes = [vp, sz, vp]
        L.or_matrix_q8_0_data.argtypes = [vp, vp, vp]
        L.or_matrix_q8_0x4_blocks.argtypes = [vp, vp]
        L.or_matrix_to_row_major.argtypes = [vp, vp, vp]
        L.or_gemv_into.argtypes = [vp, vp, vp]
        L.or_project_cpu.argtypes = [vp, vp, sz, vp]
        L.or_logits_cpu.argtypes = [vp, vp, sz, vp]
        L.or_block_dots.argtypes = [vp, vp, sz, vp]
        L.or_weights_new.restype = vp
        L.or_weights_new.argtypes = [sz]
        L.or_weights_free.argtypes = [vp]
        L.or_weights_set_embedding.argtypes = [vp, vp]
        L.or_weights_set_classifier.argtypes = [vp, vp]
        L.or_weights_set_proj.argtypes = [vp, sz, C.c_int, vp]
        L.or_weights_set_norm.argtypes = [vp, sz, C.c_int, vp, sz]
        L.or_weights_set_final_norm.argtypes = [vp, vp, sz]
        L.or_weights_set_conv.argtypes = [vp, sz, vp, sz, sz]
        L.or_llama_new.argtypes = [C.POINTER(OracleConfig), vp, C.c_char_p, C.POINTER(vp)]
        L.or_lfm2_new.argtypes = [C.POINTER(OracleConfig), vp, vp, C.c_char_p, C.POINTER(vp)]
        L.or_model_free.argtypes = [vp]
        L.or_model_kv_fill.argtypes = [vp, sz, C.c_uint64]
        L.or_model_kv_upload.argtypes = [vp, C.c_int, sz, vp, sz]
        L.or_model_forward.argtypes = [vp, sz, sz, vp, sz]
        L.or_model_prefill.argtypes = [vp, vp, sz, sz, vp, sz]
        L.or_llama_prefill_multi.argtypes = [vp, vp, vp, sz, vp, sz]
        L.or_llama_prefill_shared.argtypes = [vp, vp, sz, vp, vp, sz, vp, sz]
        L.or_backend_new.argtypes = [C.c_char_p, vp, sz, sz, sz, C.POINTER(vp)]
        L.or_backend_free.argtypes = [vp]
        L.or_b_alloc.restype = sz
        L.or_b_alloc.argtypes = [vp, sz]
        L.or_b_upload.restype = sz
        L.or_b_upload.argtypes = [vp, vp, sz]
        L.or_b_read.argtypes = [vp, sz, vp, sz]
        L.or_b_embed.argtypes = [vp, sz, sz, sz]
        L.or_b_copy.argtypes = [vp, sz, sz, sz, sz, sz]
        L.or_b_rms_norm.argtypes = [vp, sz, sz, sz, sz, sz, C.c_float]
        L.or_b_qk_norm.argtypes = [vp, sz, sz, sz, sz, sz, C.c_float]
        L.or_b_rope.argtypes = [vp, sz, sz, sz, sz, sz, vp, sz, C.c_float, C.c_int]
        L.or_b_project.argtypes = [vp, sz, C.c_int, sz, sz, sz]
        L.or_b_kv_write.argtypes = [vp, sz, vp, sz, sz, sz]
        L.or_b_attention.argtypes = [vp, sz, sz, sz, sz, vp, sz, sz, sz, sz, sz, sz]
        L.or_b_add_in_place.argtypes = [vp, sz, sz, sz]
        L.or_b_mul.argtypes = [vp, sz, sz, sz, sz, sz, sz, sz]
        L.or_b_conv_prefill.argtypes = [vp, sz, sz, sz, sz, sz, sz]
        L.or_b_conv_decode.argtypes = [vp, sz, sz, sz, sz, sz, sz]
        L.or_b_silu_mul.argtypes = [vp, sz, sz, sz]
        L.or_b_logits.argtypes = [vp, sz, sz]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _check(rc: int):
    if rc != 0:
        raise RuntimeError(lib().or_last_error().decode())


# ---- scalar helpers ---------------------------------------------------------

def f32_to_f16_bits(v: float) -> int:
    return int(lib().or_f32_to_f16_bits(float(v)))


def f16_scale_to_f32(bits: int) -> float:
    return float(lib().or_f16_scale_to_f32(int(bits)))


def expf(x: float) -> float:
    return float(lib().or_expf(float(x)))


def lcg_fill(count: int, seed: int) -> np.ndarray:
    """tests/backends.rs:41-51: the reference tests' deterministic LCG fill."""
    out = np.empty(count, dtype=np.float32)
    lib().or_lcg_fill(count, seed, _ptr(out))
    return out


def quantize(x: np.ndarray):
    """Q8Vec::quantize (quant.rs:831-851) -> (quants i8, scales f32, scales_f16 u16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = (x.size + 31) // 32
    q = np.zeros(nb * 32, dtype=np.int8)
    s = np.zeros(nb, dtype=np.float32)
    h = np.zeros(nb, dtype=np.uint16)
    lib().or_quantize(_ptr(x), x.size, _ptr(q), _ptr(s), _ptr(h))
    return q, s, h


def dot_q8_0_scalar(a, a_scales, b, b_scales) -> float:
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    sa = np.ascontiguousarray(a_scales, np.float32)
    sb = np.ascontiguousarray(b_scales, np.float32)
    return float(lib().or_dot_q8_0_scalar(_ptr(a), _ptr(sa), _ptr(b), _ptr(sb), min(sa.size, sb.size)))


def dot_scalar(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return float(lib().or_dot_scalar(_ptr(a), _ptr(b), a.size))


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().or_argmax(_ptr(v), v.size))


def softmax(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().or_softmax(_ptr(x), x.size)
    return x


# ---- matrices ---------------------------------------------------------------

class Matrix:
    """One weight matrix in a reference storage (quant.rs:502-520)."""

    def __init__(self, data: np.ndarray, storage: str):
        data = np.ascontiguousarray(data, dtype=np.float32)
        assert data.ndim == 2
        h = C.c_void_p()
        _check(lib().or_matrix_from_f32(_ptr(data), data.shape[0], data.shape[1], KIND[storage], C.byref(h)))
        self.h = h
        self.out_dim, self.in_dim = data.shape
        self.storage = storage

    @staticmethod
    def from_q8_0(quants, scales, out_dim, in_dim) -> "Matrix":
        m = Matrix.__new__(Matrix)
        q = np.ascontiguousarray(quants, np.int8)
        s = np.ascontiguousarray(scales, np.float32)
        h = C.c_void_p()
        _check(lib().or_matrix_from_q8_0(_ptr(q), _ptr(s), out_dim, in_dim, C.byref(h)))
        m.h, m.out_dim, m.in_dim, m.storage = h, out_dim, in_dim, "q8_0"
        return m

    @staticmethod
    def from_q8_0x4_blocks(blocks, out_dim, in_dim) -> "Matrix":
        m = Matrix.__new__(Matrix)
        b = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        _check(lib().or_matrix_from_q8_0x4_blocks(_ptr(b), out_dim, in_dim, C.byref(h)))
        m.h, m.out_dim, m.in_dim, m.storage = h, out_dim, in_dim, "q8_0x4"
        return m

    @staticmethod
    def try_new(data, storage):
        try:
            return Matrix(data, storage)
        except RuntimeError:
            return None

    def __del__(self):
        if getattr(self, "h", None) is not None and _lib is not None:
            _lib.or_matrix_free(self.h)
            self.h = None

    def decode_row(self, row: int) -> np.ndarray:
        out = np.empty(self.in_dim, np.float32)
        lib().or_matrix_decode_row(self.h, row, _ptr(out))
        return out

    def to_f32(self) -> np.ndarray:
        return np.stack([self.decode_row(r) for r in range(self.out_dim)])

    def q8_0_data(self):
        q = np.empty(self.out_dim * self.in_dim, np.int8)
        s = np.empty(self.out_dim * self.in_dim // 32, np.float32)
        _check(lib().or_matrix_q8_0_data(self.h, _ptr(q), _ptr(s)))
        return q, s

    def q8_0x4_blocks(self) -> np.ndarray:
        n = (self.out_dim // 4) * (self.in_dim // 32) * 136
        out = np.empty(n, np.uint8)
        _check(lib().or_matrix_q8_0x4_blocks(self.h, _ptr(out)))
        return out

    def to_row_major(self):
        q = np.empty(self.out_dim * self.in_dim, np.int8)
        s = np.empty(self.out_dim * self.in_dim // 32, np.float32)
        _check(lib().or_matrix_to_row_major(self.h, _ptr(q), _ptr(s)))
        return q, s

    def gemv(self, x) -> np.ndarray:
        """gemv_into (quant.rs:23-62)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.out_dim, np.float32)
        lib().or_gemv_into(self.h, _ptr(x), _ptr(y))
        return y

    def project_cpu(self, x) -> np.ndarray:
        """Cpu::project on this matrix (cpu.rs:304-371, prefill_f32 off)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.in_dim)
        y = np.empty((x.shape[0], self.out_dim), np.float32)
        _check(lib().or_project_cpu(self.h, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def logits_cpu(self, x) -> np.ndarray:
        """Cpu::logits on this matrix as classifier (cpu.rs:501-514)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.out_dim, np.float32)
        _check(lib().or_logits_cpu(self.h, _ptr(x), x.size, _ptr(y)))
        return y

    def block_dots(self, xq: np.ndarray) -> np.ndarray:
        xq = np.ascontiguousarray(xq, np.int8).reshape(-1, self.in_dim)
        out = np.empty((xq.shape[0], self.out_dim, self.in_dim // 32), np.int32)
        _check(lib().or_block_dots(self.h, _ptr(xq), xq.shape[0], _ptr(out)))
        return out


# ---- models -----------------------------------------------------------------

@dataclass
class Config:
    """arch/llm/llama.rs:26-67."""
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    seq_len: int
    rms_eps: float
    rope_theta: float
    rope_interleaved: bool
    head_dim: int

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    @property
    def kv_mul(self):
        return self.n_heads // self.n_kv_heads

    def to_c(self) -> OracleConfig:
        return OracleConfig(self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads,
                            self.vocab_size, self.seq_len, self.rms_eps, self.rope_theta,
                            int(self.rope_interleaved), self.head_dim)


def backends_config() -> Config:
    """tests/backends.rs:24-38."""
    return Config(dim=32, hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=32,
                  seq_len=64, rms_eps=1e-5, rope_theta=10_000.0, rope_interleaved=False, head_dim=8)


class Weights:
    """A ModelWeights (mod.rs:131-145) held in the oracle, plus the host
    copies of every tensor so the same bytes can be handed to another backend.

    ``layers[l]`` maps projection name -> Matrix and norm name -> ndarray.
    """

    def __init__(self, n_layers: int):
        self.h = lib().or_weights_new(n_layers)
        self.layers = [dict() for _ in range(n_layers)]
        self.embedding = None
        self.classifier = None
        self.final_norm = None
        self.is_attention = [True] * n_layers

    def __del__(self):
        if getattr(self, "h", None) is not None and _lib is not None:
            _lib.or_weights_free(self.h)
            self.h = None

    def set_embedding(self, m: Matrix):
        self.embedding = m
        lib().or_weights_set_embedding(self.h, m.h)

    def set_classifier(self, m):
        self.classifier = m
        lib().or_weights_set_classifier(self.h, m.h if m is not None else None)

    def set_proj(self, layer: int, name: str, m: Matrix):
        self.layers[layer][name] = m
        _check(lib().or_weights_set_proj(self.h, layer, PROJ[name], m.h))

    def set_norm(self, layer: int, which: str, v: np.ndarray):
        v = np.ascontiguousarray(v, np.float32)
        self.layers[layer]["norm_" + which] = v
        lib().or_weights_set_norm(self.h, layer, {"att": 0, "ffn": 1, "q": 2, "k": 3}[which], _ptr(v), v.size)

    def set_final_norm(self, v: np.ndarray):
        v = np.ascontiguousarray(v, np.float32)
        self.final_norm = v
        lib().or_weights_set_final_norm(self.h, _ptr(v), v.size)

    def set_conv(self, layer: int, kernel: np.ndarray):
        kernel = np.ascontiguousarray(kernel, np.float32)
        self.layers[layer]["conv_kernel"] = kernel
        self.is_attention[layer] = False
        lib().or_weights_set_conv(self.h, layer, _ptr(kernel), kernel.shape[0], kernel.shape[1])


def backends_weights(config: Config, storage: str = "f32") -> Weights:
    """tests/backends.rs:68-109 (`weights_at`), LCG fill and all."""
    dim, hidden, vocab = config.dim, config.hidden_dim, config.vocab_size

    def matrix(rows, cols, seed):
        return Matrix(lcg_fill(rows * cols, seed).reshape(rows, cols), storage)

    w = Weights(config.n_layers)
    for l in range(config.n_layers):
        s = 100 * (l + 1)
        w.set_norm(l, "att", lcg_fill(dim, s + 1))
        w.set_proj(l, "q", matrix(config.q_dim, dim, s + 2))
        w.set_proj(l, "k", matrix(config.kv_dim, dim, s + 3))
        w.set_proj(l, "v", matrix(config.kv_dim, dim, s + 4))
        w.set_proj(l, "o", matrix(dim, config.q_dim, s + 5))
        w.set_norm(l, "ffn", lcg_fill(dim, s + 6))
        w.set_proj(l, "gate", matrix(hidden, dim, s + 7))
        w.set_proj(l, "down", matrix(dim, hidden, s + 8))
        w.set_proj(l, "up", matrix(hidden, dim, s + 9))
        w.set_norm(l, "q", lcg_fill(config.head_dim, s + 10))
        w.set_norm(l, "k", lcg_fill(config.head_dim, s + 11))
    w.set_embedding(matrix(vocab, dim, 1))
    w.set_final_norm(lcg_fill(dim, 2))
    w.set_classifier(matrix(vocab, dim, 3))
    return w


def lfm2_config() -> Config:
    """src/arch/llm/lfm2.rs:660-674."""
    return Config(dim=32, hidden_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=32,
                  seq_len=64, rms_eps=1e-5, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=8)


def lfm2_weights(config: Config, mask, storage: str = "f32") -> Weights:
    """src/arch/llm/lfm2.rs:705-766 (`weights_at`), generalised to any storage."""
    dim, hidden, vocab = config.dim, config.hidden_dim, config.vocab_size

    def matrix(rows, cols, seed):
        return Matrix(lcg_fill(rows * cols, seed).reshape(rows, cols), storage)

    w = Weights(config.n_layers)
    for l, attn in enumerate(mask):
        s = 100 * (l + 1)
        if attn:
            w.set_proj(l, "q", matrix(config.q_dim, dim, s + 2))
            w.set_proj(l, "k", matrix(config.kv_dim, dim, s + 3))
            w.set_proj(l, "v", matrix(config.kv_dim, dim, s + 4))
            w.set_proj(l, "o", matrix(dim, config.q_dim, s + 5))
            w.set_norm(l, "q", lcg_fill(config.head_dim, s + 10))
            w.set_norm(l, "k", lcg_fill(config.head_dim, s + 11))
        else:
            w.set_proj(l, "conv_in", matrix(3 * dim, dim, s + 12))
            w.set_proj(l, "conv_out", matrix(dim, dim, s + 13))
            w.set_conv(l, lcg_fill(dim * 3, s + 14).reshape(dim, 3))
        w.set_norm(l, "att", lcg_fill(dim, s + 1))
        w.set_norm(l, "ffn", lcg_fill(dim, s + 6))
        w.set_proj(l, "gate", matrix(hidden, dim, s + 7))
        w.set_proj(l, "down", matrix(dim, hidden, s + 8))
        w.set_proj(l, "up", matrix(hidden, dim, s + 9))
    w.set_embedding(matrix(vocab, dim, 1))
    w.set_final_norm(lcg_fill(dim, 2))
    w.set_classifier(None)
    return w


class Model:
    """Llama (llama.rs:169-863) or Lfm2 (lfm2.rs:118-641) over the oracle."""

    def __init__(self, config: Config, weights: Weights, backend: str = "cpu", lfm2: bool = False):
        self.config = config
        self.weights = weights  # keep alive
        h = C.c_void_p()
        cc = config.to_c()
        if lfm2:
            mask = (C.c_int * config.n_layers)(*[int(a) for a in weights.is_attention])
            _check(lib().or_lfm2_new(C.byref(cc), mask, weights.h, backend.encode(), C.byref(h)))
        else:
            _check(lib().or_llama_new(C.byref(cc), weights.h, backend.encode(), C.byref(h)))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None) is not None and _lib is not None:
            _lib.or_model_free(self.h)
            self.h = None

    def kv_fill(self, slots: int, seed: int):
        """Benchmark set-up: N(0,1) into cache slots [0, slots) of every layer."""
        _check(lib().or_model_kv_fill(self.h, slots, seed))

    def kv_upload(self, which: int, offset: int, data):
        """Test set-up: values into the key (0) or value (1) cache at an element
        offset of [n_layers, seq_len, kv_dim]."""
        d = np.ascontiguousarray(data, np.float32)
        _check(lib().or_model_kv_upload(self.h, which, offset, _ptr(d), d.size))

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.config.vocab_size, np.float32)
        _check(lib().or_model_forward(self.h, token, pos, _ptr(out), out.size))
        return out

    def prefill(self, tokens, start: int = 0) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint64)
        out = np.empty(self.config.vocab_size, np.float32)
        _check(lib().or_model_prefill(self.h, _ptr(t), t.size, start, _ptr(out), out.size))
        return out

    def prefill_multi(self, seqs):
        flat = np.ascontiguousarray([t for s in seqs for t in s], np.uint64)
        lens = np.ascontiguousarray([len(s) for s in seqs], np.uint64)
        out = np.zeros((len(seqs), self.config.dim), np.float32)
        _check(lib().or_llama_prefill_multi(self.h, _ptr(flat), _ptr(lens), len(seqs), _ptr(out), self.config.dim))
        return out

    def prefill_shared(self, prefix, suffixes):
        p = np.ascontiguousarray(prefix, np.uint64)
        flat = np.ascontiguousarray([t for s in suffixes for t in s], np.uint64)
        lens = np.ascontiguousarray([len(s) for s in suffixes], np.uint64)
        out = np.zeros((len(suffixes), self.config.dim), np.float32)
        _check(lib().or_llama_prefill_shared(self.h, _ptr(p), p.size, _ptr(flat), _ptr(lens), len(suffixes),
                                             _ptr(out), self.config.dim))
        return out


class Backend:
    """A bare oracle backend (cpu.rs / reference.rs) for op-level checks."""

    def __init__(self, name: str = "cpu", weights: Weights | None = None, n_layers: int = 0,
                 kv_dim: int = 0, seq_len: int = 0):
        h = C.c_void_p()
        _check(lib().or_backend_new(name.encode(), weights.h if weights else None, n_layers, kv_dim, seq_len,
                                    C.byref(h)))
        self.h = h
        self.weights = weights

    def __del__(self):
        if getattr(self, "h", None) is not None and _lib is not None:
            _lib.or_backend_free(self.h)
            self.h = None

    def alloc(self, n):
        return lib().or_b_alloc(self.h, n)

    def upload(self, data):
        d = np.ascontiguousarray(data, np.float32)
        return lib().or_b_upload(self.h, _ptr(d), d.size)

    def read(self, buf, n):
        out = np.empty(n, np.float32)
        lib().or_b_read(self.h, buf, _ptr(out), n)
        return out

    def embed(self, token, out, offset):
        _check(lib().or_b_embed(self.h, token, out, offset))

    def copy(self, src, so, dst, do, n):
        lib().or_b_copy(self.h, src, so, dst, do, n)

    def rms_norm(self, out, x, w, rows, dim, eps):
        lib().or_b_rms_norm(self.h, out, x, w, rows, dim, eps)

    def qk_norm(self, v, rows, width, head, w, eps):
        lib().or_b_qk_norm(self.h, v, rows, width, head, w, eps)

    def rope(self, q, k, qw, kvw, rows, positions, head_size, theta, interleaved):
        p = np.ascontiguousarray(positions, np.uint64)
        lib().or_b_rope(self.h, q, k, qw, kvw, rows, _ptr(p), head_size, theta, int(interleaved))

    def project(self, layer, proj, x, y, rows):
        _check(lib().or_b_project(self.h, layer, PROJ[proj] if isinstance(proj, str) else proj, x, y, rows))

    def kv_write(self, layer, slots, k, v, rows):
        s = np.ascontiguousarray(slots, np.uint64)
        lib().or_b_kv_write(self.h, layer, _ptr(s), k, v, rows)

    def attention(self, q, out, att, layer, windows, n_heads, kv_mul, head_size, kv_dim, seq_len):
        ws = (OracleWindow * len(windows))(*[OracleWindow(*w) for w in windows])
        lib().or_b_attention(self.h, q, out, att, layer, ws, len(windows), n_heads, kv_mul, head_size, kv_dim,
                             seq_len)

    def add_in_place(self, d, s, n):
        lib().or_b_add_in_place(self.h, d, s, n)

    def mul(self, o, oo, a, ao, b, bo, n):
        lib().or_b_mul(self.h, o, oo, a, ao, b, bo, n)

    def conv_prefill(self, o, x, kern, rows, dim, k):
        lib().or_b_conv_prefill(self.h, o, x, kern, rows, dim, k)

    def conv_decode(self, o, x, kern, state, dim, k):
        lib().or_b_conv_decode(self.h, o, x, kern, state, dim, k)

    def silu_mul(self, g, u, n):
        lib().or_b_silu_mul(self.h, g, u, n)

    def logits(self, x, y):
        _check(lib().or_b_logits(self.h, x, y))
