"""Python mirror of KernRT's backend seam (src/backends/mod.rs) over the HIP
backend's C ABI (include/kernrt_hip.h).

Same names, argument meanings and error behaviour as the reference trait:
buffers are integer handles (`Buf`), every op may be deferred, `read` is the
barrier, `open` raises `BackendError` (with `detail` set when the backend
exists but cannot start) and misuse of an op raises (the reference panics).
"""

from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import KrAttnSpec, KrRopeSpec, KrWindow

Buf = int

# Proj::index (mod.rs:100-112)
PROJ_INDEX = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "down": 5, "up": 6, "conv_in": 7, "conv_out": 8}
PROJ_ALL = tuple(PROJ_INDEX)

STORAGE_Q8_0 = 2
STORAGE_Q8_0X4 = 3
KR_NO_MAT = 0xFFFFFFFF
KR_NO_BUF = 0xFFFFFFFF


class BackendError(Exception):
    """mod.rs:190-213: `detail` is set when the backend exists but refused to start."""

    def __init__(self, requested: str, detail: Optional[str] = None):
        self.requested = requested
        self.detail = detail
        super().__init__(str(self))

    def __str__(self):
        if self.detail is not None:
            return f"backend {self.requested!r} is unavailable: {self.detail}"
        return f"unknown backend {self.requested!r}; available: {', '.join(available())}"


def available() -> list[str]:
    """mod.rs:216-225: the names `open` accepts."""
    return ["hip"]


def open(name: str) -> "Hip":
    """mod.rs:228-244: build a backend by name."""
    if name == "hip":
        return Hip()
    raise BackendError(name, None)


def from_env() -> "Hip":
    """mod.rs:247-252: KERNRT_BACKEND, defaulting to the one arm this package has."""
    name = os.environ.get("KERNRT_BACKEND", "hip").strip() or "hip"
    return open(name)


@dataclass
class RopeSpec:  # mod.rs:149-155
    head_size: int
    theta: float
    interleaved: bool


@dataclass
class AttnSpec:  # mod.rs:158-167
    n_heads: int
    kv_mul: int
    head_size: int
    kv_dim: int
    seq_len: int


@dataclass
class KvSpec:  # mod.rs:170-177
    n_layers: int
    kv_dim: int
    seq_len: int


@dataclass
class Window:  # mod.rs:181-188
    att_start: int
    slot: int
    shared: tuple = (0, 0)


@dataclass
class Q8Matrix:
    """One quantized weight matrix as the loader holds it (quant.rs:502-520).

    storage "q8_0": `quants` int8 [out*in] and `scales` f32 [out*in/32];
    storage "q8_0x4": `blocks` uint8 [(out/4)*(in/32)*136] (Q8Block4 records).
    """
    storage: str
    out_dim: int
    in_dim: int
    quants: Optional[np.ndarray] = None
    scales: Optional[np.ndarray] = None
    blocks: Optional[np.ndarray] = None


@dataclass
class SourceMatrix:
    """A checkpoint weight matrix in the storage the loader chose for it
    (`matrix_from_raw`, hf.rs:151-200). `kind` is the reference's
    `Matrix::kind()` (quant.rs:565-572): "q8_0" / "q8_0x4" carry the f32 values
    or bf16 bit patterns they are quantized from, on the device, at upload
    (`kr_matrix_quantize`); "f32" / "bf16" carry the values themselves, which
    this backend does not hold."""
    kind: str
    out_dim: int
    in_dim: int
    values: np.ndarray  # flat float32, or uint16 bf16 bits

    @property
    def storage(self) -> str:
        return self.kind


@dataclass
class LayerWeights:  # formats/llama2c.rs:49-76
    rms_att: np.ndarray
    rms_ffn: np.ndarray
    proj: dict = field(default_factory=dict)  # name -> Q8Matrix
    rms_q: Optional[np.ndarray] = None
    rms_k: Optional[np.ndarray] = None
    conv_kernel: Optional[np.ndarray] = None  # [dim, k]
    is_attention: bool = True


@dataclass
class ModelWeights:  # mod.rs:131-145
    token_embedding: Q8Matrix
    layers: list
    rms_final: np.ndarray
    wcls: Optional[Q8Matrix] = None


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def q8_0x4_records(quants: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """The reference's Q8_0x4 storage (`Q8Block4`, quant.rs:113-118) of a
    row-major int8 matrix [out_dim, in_dim] and its f16 scale bits
    [out_dim, in_dim / 32]: (out_dim / 4) x (in_dim / 32) records of 136
    bytes, {u16 scales[4]; i8 quants[128]} with quants[seg * 16 + r * 4 + lane]
    = row 4 g + r, column 32 b + 4 seg + lane -- the inverse of the
    de-interleave kr_matrix_q8_0x4 does on upload."""
    n, k = quants.shape
    g, nb = n // 4, k // 32
    q = np.ascontiguousarray(quants, np.int8).reshape(g, 4, nb, 8, 4).transpose(0, 2, 3, 1, 4).reshape(g, nb, 128)
    s = np.ascontiguousarray(scales_f16, np.uint16).reshape(g, 4, nb).transpose(0, 2, 1)
    rec = np.empty((g, nb, 136), np.uint8)
    rec[:, :, :8] = np.ascontiguousarray(s).view(np.uint8).reshape(g, nb, 8)
    rec[:, :, 8:] = q.view(np.uint8)
    return rec.ravel()


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Hip:
    """The `hip` backend: one device, one stream, `read` is the barrier."""

    def __init__(self, device: int = 0):
        self._L = _lib.load()
        ctx = C.c_void_p()
        detail = C.create_string_buffer(256)
        rc = self._L.kr_open(device, C.byref(ctx), detail, 256)
        if rc != 0:
            raise BackendError("hip", detail.value.decode() or f"open failed ({rc})")
        self.ctx = ctx
        self._weights_bound = False
        self._models = weakref.WeakSet()  # drivers borrowing this context

    def close(self):
        if getattr(self, "ctx", None):
            for m in list(self._models):  # a driver must not outlive its backend
                m.close()
            self._L.kr_close(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ck(self, rc: int):
        if rc != 0:
            raise RuntimeError(self._L.kr_last_error(self.ctx).decode())

    # ---- identity
    def name(self) -> str:
        return self._L.kr_name(self.ctx).decode()

    def storage(self) -> str:
        return self._L.kr_storage(self.ctx).decode()

    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        self._ck(self._L.kr_device_name(self.ctx, buf, 256))
        return buf.value.decode()

    # ---- weights
    def upload_matrix(self, m) -> int:
        h = C.c_uint32()
        if isinstance(m, SourceMatrix):
            if m.kind not in ("q8_0", "q8_0x4"):
                raise RuntimeError(f"the hip backend stores Q8_0/Q8_0x4 weights only, not {m.kind} "
                                   "(KERNRT_Q8_0=1 or KERNRT_Q8_0X4=1 loads a checkpoint as Q8)")
            v = m.values
            if v.dtype == np.uint16:
                src = _lib.SRC_BF16
            else:
                src, v = _lib.SRC_F32, _f32(v)
            v = np.ascontiguousarray(v)
            if v.size != m.out_dim * m.in_dim:
                raise ValueError(f"matrix [{m.out_dim}, {m.in_dim}] given {v.size} values")
            kind = STORAGE_Q8_0 if m.kind == "q8_0" else STORAGE_Q8_0X4
            self._ck(self._L.kr_matrix_quantize(self.ctx, kind, src, _p(v), m.out_dim, m.in_dim, C.byref(h)))
        elif m.storage == "q8_0":
            q = np.ascontiguousarray(m.quants, np.int8)
            s = _f32(m.scales)
            self._ck(self._L.kr_matrix_q8_0(self.ctx, m.out_dim, m.in_dim, _p(q), _p(s), C.byref(h)))
        elif m.storage == "q8_0x4":
            b = np.ascontiguousarray(m.blocks, np.uint8)
            self._ck(self._L.kr_matrix_q8_0x4(self.ctx, m.out_dim, m.in_dim, _p(b), C.byref(h)))
        else:
            raise RuntimeError(f"the hip backend stores Q8_0/Q8_0x4 weights only, not {m.storage}")
        return h.value

    def synthetic_matrix(self, storage: str, out_dim: int, in_dim: int, seed: int, stddev: float = 0.02) -> int:
        h = C.c_uint32()
        kind = STORAGE_Q8_0 if storage == "q8_0" else STORAGE_Q8_0X4
        self._ck(self._L.kr_matrix_synthetic(self.ctx, kind, out_dim, in_dim, seed, stddev, C.byref(h)))
        return h.value

    def free_matrix(self, h: int):
        self._ck(self._L.kr_matrix_free(self.ctx, h))

    def bind_weights(self, w: ModelWeights):
        """Upload and bind every matrix of `w` (the first half of `prepare`)."""
        emb = self.upload_matrix(w.token_embedding)
        self._ck(self._L.kr_bind_embedding(self.ctx, emb))
        cls = self.upload_matrix(w.wcls) if w.wcls is not None else KR_NO_MAT
        self._ck(self._L.kr_bind_classifier(self.ctx, cls))
        for l, layer in enumerate(w.layers):
            for name, m in layer.proj.items():
                self._ck(self._L.kr_bind_proj(self.ctx, l, PROJ_INDEX[name], self.upload_matrix(m)))
        self._weights_bound = True

    def bind_handles(self, embedding: int, classifier: int, layers: Sequence[dict]):
        self._ck(self._L.kr_bind_embedding(self.ctx, embedding))
        self._ck(self._L.kr_bind_classifier(self.ctx, classifier))
        for l, projs in enumerate(layers):
            for name, h in projs.items():
                self._ck(self._L.kr_bind_proj(self.ctx, l, PROJ_INDEX[name], h))
        self._weights_bound = True

    def prepare(self, weights: Optional[ModelWeights], kv: KvSpec):
        """mod.rs:272: upload/bind weights (unless already bound) and size the cache."""
        if weights is not None and not self._weights_bound:
            self.bind_weights(weights)
        self._ck(self._L.kr_prepare(self.ctx, kv.n_layers, kv.kv_dim, kv.seq_len))

    # ---- memory (mod.rs:274-282)
    def alloc(self, n: int) -> Buf:
        h = C.c_uint32()
        self._ck(self._L.kr_alloc(self.ctx, n, C.byref(h)))
        return h.value

    def upload(self, data) -> Buf:
        d = _f32(data).ravel()
        h = C.c_uint32()
        self._ck(self._L.kr_upload(self.ctx, _p(d), d.size, C.byref(h)))
        return h.value

    def read(self, src: Buf, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self._ck(self._L.kr_read(self.ctx, src, _p(out), n))
        return out

    # ---- ops (mod.rs:284-403)
    def embed(self, token: int, out: Buf, offset: int):
        self._ck(self._L.kr_embed(self.ctx, token, out, offset))

    def copy(self, src: Buf, src_offset: int, dst: Buf, dst_offset: int, n: int):
        self._ck(self._L.kr_copy(self.ctx, src, src_offset, dst, dst_offset, n))

    def rms_norm(self, out: Buf, x: Buf, weight: Buf, rows: int, dim: int, eps: float):
        self._ck(self._L.kr_rms_norm(self.ctx, out, x, weight, rows, dim, eps))

    def qk_norm(self, v: Buf, rows: int, width: int, head_size: int, weight: Buf, eps: float):
        self._ck(self._L.kr_qk_norm(self.ctx, v, rows, width, head_size, weight, eps))

    def rope(self, q: Buf, k: Buf, q_width: int, kv_width: int, rows: int, positions, spec: RopeSpec):
        p = np.ascontiguousarray(positions, np.uint64)
        s = KrRopeSpec(spec.head_size, spec.theta, int(spec.interleaved))
        self._ck(self._L.kr_rope(self.ctx, q, k, q_width, kv_width, rows, _p(p), C.byref(s)))

    def project(self, layer: int, proj: str, x: Buf, y: Buf, rows: int):
        self._ck(self._L.kr_project(self.ctx, layer, PROJ_INDEX[proj], x, y, rows))

    def project_qkv(self, layer: int, x: Buf, q: Buf, k: Buf, v: Buf, rows: int):
        self._ck(self._L.kr_project_qkv(self.ctx, layer, x, q, k, v, rows))

    def project_gate_up(self, layer: int, x: Buf, gate: Buf, up: Buf, rows: int):
        self._ck(self._L.kr_project_gate_up(self.ctx, layer, x, gate, up, rows))

    def kv_write(self, layer: int, slots, k: Buf, v: Buf, rows: int):
        s = np.ascontiguousarray(slots, np.uint64)
        self._ck(self._L.kr_kv_write(self.ctx, layer, _p(s), k, v, rows))

    def attention(self, q: Buf, out: Buf, att: Buf, layer: int, windows: Sequence[Window], spec: AttnSpec):
        ws = (KrWindow * max(len(windows), 1))(*[KrWindow(w.att_start, w.slot, w.shared[0], w.shared[1])
                                                  for w in windows])
        s = KrAttnSpec(spec.n_heads, spec.kv_mul, spec.head_size, spec.kv_dim, spec.seq_len)
        self._ck(self._L.kr_attention(self.ctx, q, out, att, layer, ws, len(windows), C.byref(s)))

    def add_in_place(self, dst: Buf, src: Buf, n: int):
        self._ck(self._L.kr_add_in_place(self.ctx, dst, src, n))

    def mul(self, out: Buf, out_off: int, a: Buf, a_off: int, b: Buf, b_off: int, n: int):
        self._ck(self._L.kr_mul(self.ctx, out, out_off, a, a_off, b, b_off, n))

    def conv_prefill(self, out: Buf, x: Buf, kernel: Buf, rows: int, dim: int, k: int):
        self._ck(self._L.kr_conv_prefill(self.ctx, out, x, kernel, rows, dim, k))

    def conv_decode(self, out: Buf, x: Buf, kernel: Buf, state: Buf, dim: int, k: int):
        self._ck(self._L.kr_conv_decode(self.ctx, out, x, kernel, state, dim, k))

    def silu_mul(self, gate: Buf, up: Buf, n: int):
        self._ck(self._L.kr_silu_mul(self.ctx, gate, up, n))

    def logits(self, x: Buf, y: Buf):
        self._ck(self._L.kr_logits(self.ctx, x, y))

    # ---- unbound-matrix kernels and parity probes
    def matmul(self, mat: int, x: Buf, y: Buf, rows: int):
        self._ck(self._L.kr_matmul(self.ctx, mat, x, y, rows))

    def matmul_noalloc(self, mat: int, x: Buf, y: Buf, rows: int):
        """`matmul` through the entry point that allocates nothing
        (kr_matmul_noalloc): rows * in_dim <= matmul_noalloc_max_elems()."""
        self._ck(self._L.kr_matmul_noalloc(self.ctx, mat, x, y, rows))

    def matmul_noalloc_max_elems(self) -> int:
        return int(self._L.kr_matmul_noalloc_max_elems())

    def quantize_rows(self, x: Buf, rows: int, width: int):
        self._ck(self._L.kr_quantize_rows(self.ctx, x, rows, width))

    def matmul_quantized(self, mat: int, y: Buf, rows: int):
        self._ck(self._L.kr_matmul_quantized(self.ctx, mat, y, rows))

    def matmul_quantized_set(self, mats, ys, rows: int):
        """One fused launch over 1-3 matrices with the same in_dim (the kernel
        behind project_qkv / project_gate_up), on the quantized workspace."""
        n = len(mats)
        ws = (C.c_uint32 * n)(*mats)
        yb = (C.c_uint32 * n)(*ys)
        self._ck(self._L.kr_matmul_quantized_set(self.ctx, ws, yb, n, rows))

    def matmul_split(self, mat: int, x, y: Buf, rows: int):
        """The chain-split projection: y (4 * rows * out_dim floats) gets the
        four partial-sum planes; x None reuses the workspace rows of the last
        call."""
        self._ck(self._L.kr_matmul_split(self.ctx, mat, KR_NO_BUF if x is None else x, y, rows))

    def stream_read(self, src: Buf, offset: int, n: int, chunks_per_lane: int = 2, workgroups: int = 0):
        """Read n floats of src and discard them (a bandwidth reference):
        chunks_per_lane 16-byte loads per lane per round on `workgroups`
        workgroups (0: one round each)."""
        self._ck(self._L.kr_stream_read_shape(self.ctx, src, offset, n, chunks_per_lane, workgroups))

    def capture_begin(self):
        """Record the following ops into one HIP graph instead of running them."""
        self._ck(self._L.kr_capture_begin(self.ctx))

    def capture_end(self):
        self._ck(self._L.kr_capture_end(self.ctx))

    def replay(self, times: int = 1):
        """Launch the captured graph `times` times on the context's stream."""
        self._ck(self._L.kr_replay(self.ctx, times))

    def timer_start(self):
        self._ck(self._L.kr_timer_start(self.ctx))

    def timer_stop(self) -> float:
        """Milliseconds since timer_start, measured by events on the stream."""
        ms = C.c_float()
        self._ck(self._L.kr_timer_stop(self.ctx, C.byref(ms)))
        return ms.value

    def classify(self, mat: int, x: Buf, y: Buf):
        self._ck(self._L.kr_classify(self.ctx, mat, x, y))

    def dbg_quantize(self, x: Buf, rows: int, width: int):
        q = np.empty(rows * width, np.int8)
        s = np.empty(rows * width // 32, np.float32)
        h = np.empty(rows * width // 32, np.uint16)
        self._ck(self._L.kr_dbg_quantize(self.ctx, x, rows, width, _p(q), _p(s), _p(h)))
        return q, s, h

    def dbg_block_dots(self, mat: int, x: Buf, rows: int, out_dim: int, in_dim: int) -> np.ndarray:
        out = np.empty((rows, out_dim, in_dim // 32), np.int32)
        self._ck(self._L.kr_dbg_block_dots(self.ctx, mat, x, rows, _p(out)))
        return out

    def kv_upload(self, which: int, offset: int, data):
        d = _f32(data).ravel()
        self._ck(self._L.kr_kv_upload(self.ctx, which, offset, _p(d), d.size))

    def kv_read(self, which: int, offset: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self._ck(self._L.kr_kv_read(self.ctx, which, offset, _p(out), n))
        return out

    def mfma_rate(self, kind: int, workgroups: int, iters: int) -> float:
        """Launch the int8 MFMA probe (kr_mfma_rate); returns the ops issued."""
        ops = C.c_double()
        self._ck(self._L.kr_mfma_rate(self.ctx, kind, workgroups, iters, C.byref(ops)))
        return ops.value

    def synthetic_values(self, n: int, seed: int, stddev: float = 0.02) -> np.ndarray:
        """The f32 values synthetic_matrix(seed, stddev) quantizes, flattened."""
        b = self.alloc(n)
        self._ck(self._L.kr_synthetic_values(self.ctx, b, n, seed, stddev))
        return self.read(b, n)

    def dbg_mfma_f32(self, a, b, acc) -> np.ndarray:
        """kr_dbg_mfma_f32: a, b [groups, 64], acc [groups, 32, 64] -> out like acc."""
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        acc = np.ascontiguousarray(acc, np.float32)
        out = np.empty_like(acc)
        self._ck(self._L.kr_dbg_mfma_f32(self.ctx, _p(a), _p(b), _p(acc), _p(out), a.shape[0]))
        return out

    def dbg_serial_sum(self, values, waves: int = 1):
        """kr_dbg_serial_sum: values [count, n] summed by the parallel exact
        form over `waves` waves and by the chain -> (fast sums, fast applied,
        chain sums, fast clocks, chain clocks), each [count]."""
        v = np.ascontiguousarray(values, np.float32)
        if v.ndim != 2:
            raise ValueError("values must be [count, n]")
        out = np.empty((v.shape[0], 5), np.uint32)
        self._ck(self._L.kr_dbg_serial_sum(self.ctx, _p(v), v.shape[1], v.shape[0], waves, _p(out)))
        return (out[:, 0].view(np.float32).copy(), out[:, 1].astype(bool), out[:, 2].view(np.float32).copy(),
                out[:, 3].copy(), out[:, 4].copy())

    def matrix_shape(self, mat: int):
        """(storage, out_dim, in_dim) of a device matrix."""
        n, k, st = C.c_size_t(), C.c_size_t(), C.c_int()
        self._ck(self._L.kr_matrix_shape(self.ctx, mat, C.byref(n), C.byref(k), C.byref(st)))
        return ("q8_0" if st.value == STORAGE_Q8_0 else "q8_0x4"), n.value, k.value

    def read_matrix(self, mat: int, storage: str = None, out_dim: int = None, in_dim: int = None):
        """The device bytes of a matrix: int8 quants [out_dim, in_dim] and the
        block scales (f32 for q8_0, f16 bits as uint16 for q8_0x4). The shape
        comes from the library; the optional arguments are checked against it."""
        st, n, k = self.matrix_shape(mat)
        if (storage, out_dim, in_dim) != (None, None, None) and (storage, out_dim, in_dim) != (st, n, k):
            raise ValueError(f"matrix {mat} is {st} [{n}, {k}], not {storage} [{out_dim}, {in_dim}]")
        q = np.empty((n, k), np.int8)
        s = np.empty((n, k // 32), np.float32 if st == "q8_0" else np.uint16)
        self._ck(self._L.kr_matrix_read(self.ctx, mat, _p(q), q.nbytes, _p(s), s.nbytes))
        return q, s

    def kv_synthetic(self, slots: int, seed: int):
        self._ck(self._L.kr_kv_synthetic(self.ctx, slots, seed))

    def argmax(self, x: Buf, n: int, index: int = 0):
        self._ck(self._L.kr_argmax(self.ctx, x, n, index))

    def read_tokens(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint64)
        self._ck(self._L.kr_read_tokens(self.ctx, _p(out), n))
        return out

    def synchronize(self):
        self._ck(self._L.kr_synchronize(self.ctx))
