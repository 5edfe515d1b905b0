"""Python handle on the C++ model drivers (include/kernrt_llm.h), which mirror
the reference's `Llama` (src/arch/llm/llama.rs) and `Lfm2`
(src/arch/llm/lfm2.rs) over the HIP backend.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import KrlConfig, KrlLayer, KrlWeights
from .backends import Hip, ModelWeights


@dataclass
class Config:  # llama.rs:26-67
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

    def to_c(self) -> KrlConfig:
        return KrlConfig(self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads,
                         self.vocab_size, self.seq_len, self.rms_eps, self.rope_theta,
                         int(self.rope_interleaved), self.head_dim)


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


class Model:
    """`Llama` or `Lfm2` (lfm2=True) driving a `Hip` backend.

    ``weights`` may be a `ModelWeights` (matrices are uploaded and bound) or
    None when the matrices were already bound on the backend; ``norms`` then
    gives the per-layer f32 tensors.
    """

    def __init__(self, config: Config, backend: Hip, weights: Optional[ModelWeights] = None,
                 lfm2: bool = False, layers: Optional[Sequence] = None, rms_final=None):
        self.L = _lib.load()
        self.config = config
        self.backend = backend
        if weights is not None:
            backend.bind_weights(weights)
            layers = weights.layers
            rms_final = weights.rms_final
        keep = []

        def arr(a, n=None):
            if a is None:
                return None
            a = np.ascontiguousarray(a, np.float32).ravel()
            keep.append(a)
            return _p(a)

        cl = (KrlLayer * config.n_layers)()
        for l, lw in enumerate(layers):
            cl[l].rms_att = arr(lw.rms_att)
            cl[l].rms_ffn = arr(lw.rms_ffn)
            cl[l].rms_q = arr(lw.rms_q)
            cl[l].rms_k = arr(lw.rms_k)
            cl[l].conv_kernel = arr(lw.conv_kernel)
            cl[l].conv_k = 0 if lw.conv_kernel is None else np.asarray(lw.conv_kernel).shape[1]
            cl[l].is_attention = int(lw.is_attention)
        w = KrlWeights(cl, arr(rms_final))
        cfg = config.to_c()
        h = C.c_void_p()
        new = self.L.krl_lfm2_new if lfm2 else self.L.krl_llama_new
        rc = new(backend.ctx, C.byref(cfg), C.byref(w), C.byref(h))
        if rc != 0:
            raise RuntimeError(self.L.kr_last_error(backend.ctx).decode())
        self.h = h
        backend._models.add(self)

    def close(self):
        if getattr(self, "h", None):
            if getattr(self.backend, "ctx", None):  # else the backend closed us first
                self.L.krl_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ck(self, rc):
        if rc != 0:
            raise RuntimeError(self.L.krl_last_error(self.h).decode())

    def storage(self) -> str:
        return self.backend.storage()

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.config.vocab_size, np.float32)
        self._ck(self.L.krl_forward(self.h, token, pos, _p(out)))
        return out

    def prefill(self, tokens, start: int = 0) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint64)
        out = np.empty(self.config.vocab_size, np.float32)
        self._ck(self.L.krl_prefill(self.h, _p(t), t.size, start, _p(out)))
        return out

    def prefill_multi(self, seqs) -> np.ndarray:
        flat = np.ascontiguousarray([t for s in seqs for t in s], np.uint64)
        lens = np.ascontiguousarray([len(s) for s in seqs], np.uint64)
        out = np.zeros((len(seqs), self.config.dim), np.float32)
        self._ck(self.L.krl_prefill_multi(self.h, _p(flat), _p(lens), len(seqs), _p(out)))
        return out

    def decode_batch(self, tokens, rope_pos, slots, att_start, read: bool = True) -> Optional[np.ndarray]:
        """One decode step for independent sequences sharing the cache: row s
        feeds tokens[s] at RoPE position rope_pos[s] into slot slots[s] and
        attends over slots att_start[s]..=slots[s]. Returns logits [n][vocab]
        (with read=False they stay on the device and None is returned)."""
        cols = [np.ascontiguousarray(a, np.uint64) for a in (tokens, rope_pos, slots, att_start)]
        n = len(cols[0])
        assert all(len(c) == n for c in cols)
        out = np.zeros((n, self.config.vocab_size), np.float32) if read else None
        self._ck(self.L.krl_decode_batch(self.h, *(_p(c) for c in cols), n, _p(out)))
        return out

    def prefill_shared(self, prefix, suffixes) -> np.ndarray:
        p = np.ascontiguousarray(prefix, np.uint64)
        flat = np.ascontiguousarray([t for s in suffixes for t in s], np.uint64)
        lens = np.ascontiguousarray([len(s) for s in suffixes], np.uint64)
        out = np.zeros((len(suffixes), self.config.dim), np.float32)
        self._ck(self.L.krl_prefill_shared(self.h, _p(p), p.size, _p(flat), _p(lens), len(suffixes), _p(out)))
        return out

    def generate_greedy(self, token: int, pos: int, n_steps: int, use_graph: bool = True) -> np.ndarray:
        out = np.empty(n_steps, np.uint64)
        self._ck(self.L.krl_generate_greedy(self.h, token, pos, n_steps, _p(out), int(use_graph)))
        return out
