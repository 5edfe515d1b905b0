"""ctypes bindings of libkernrt_hip.so (include/kernrt_hip.h, include/kernrt_llm.h).

The library is built in-tree by kernrt_amd/build.py. Loading fails loudly when
it is missing: there is no CPU fallback behind these entry points.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkernrt_hip.so")

# kr_matrix_quantize source kinds (include/kernrt_hip.h)
SRC_F32 = 0
SRC_BF16 = 1

sz = C.c_size_t
vp = C.c_void_p
u32 = C.c_uint32
i32 = C.c_int


class KrWindow(C.Structure):
    _fields_ = [("att_start", sz), ("slot", sz), ("shared_start", sz), ("shared_end", sz)]


class KrAttnSpec(C.Structure):
    _fields_ = [("n_heads", sz), ("kv_mul", sz), ("head_size", sz), ("kv_dim", sz), ("seq_len", sz)]


class KrRopeSpec(C.Structure):
    _fields_ = [("head_size", sz), ("theta", C.c_float), ("interleaved", i32)]


class KrlConfig(C.Structure):
    _fields_ = [("dim", sz), ("hidden_dim", sz), ("n_layers", sz), ("n_heads", sz), ("n_kv_heads", sz),
                ("vocab_size", sz), ("seq_len", sz), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("rope_interleaved", i32), ("head_dim", sz)]


class KrlLayer(C.Structure):
    _fields_ = [("rms_att", vp), ("rms_ffn", vp), ("rms_q", vp), ("rms_k", vp), ("conv_kernel", vp),
                ("conv_k", sz), ("is_attention", i32)]


class KrlWeights(C.Structure):
    _fields_ = [("layers", C.POINTER(KrlLayer)), ("rms_final", vp)]


# name -> (restype, argtypes); every entry returns an int status unless noted
_SIGS = {
    "kr_open": (i32, [i32, C.POINTER(vp), C.c_char_p, sz]),
    "kr_close": (None, [vp]),
    "kr_last_error": (C.c_char_p, [vp]),
    "kr_name": (C.c_char_p, [vp]),
    "kr_storage": (C.c_char_p, [vp]),
    "kr_device_name": (i32, [vp, C.c_char_p, sz]),
    "kr_matrix_q8_0": (i32, [vp, sz, sz, vp, vp, C.POINTER(u32)]),
    "kr_matrix_q8_0x4": (i32, [vp, sz, sz, vp, C.POINTER(u32)]),
    "kr_matrix_synthetic": (i32, [vp, i32, sz, sz, C.c_uint64, C.c_float, C.POINTER(u32)]),
    "kr_matrix_quantize": (i32, [vp, i32, i32, vp, sz, sz, C.POINTER(u32)]),
    "kr_mfma_rate": (i32, [vp, i32, sz, sz, C.POINTER(C.c_double)]),
    "kr_synthetic_values": (i32, [vp, u32, sz, C.c_uint64, C.c_float]),
    "kr_matrix_free": (i32, [vp, u32]),
    "kr_bind_embedding": (i32, [vp, u32]),
    "kr_bind_classifier": (i32, [vp, u32]),
    "kr_bind_proj": (i32, [vp, sz, i32, u32]),
    "kr_prepare": (i32, [vp, sz, sz, sz]),
    "kr_alloc": (i32, [vp, sz, C.POINTER(u32)]),
    "kr_upload": (i32, [vp, vp, sz, C.POINTER(u32)]),
    "kr_read": (i32, [vp, u32, vp, sz]),
    "kr_embed": (i32, [vp, sz, u32, sz]),
    "kr_copy": (i32, [vp, u32, sz, u32, sz, sz]),
    "kr_rms_norm": (i32, [vp, u32, u32, u32, sz, sz, C.c_float]),
    "kr_qk_norm": (i32, [vp, u32, sz, sz, sz, u32, C.c_float]),
    "kr_rope": (i32, [vp, u32, u32, sz, sz, sz, vp, C.POINTER(KrRopeSpec)]),
    "kr_project": (i32, [vp, sz, i32, u32, u32, sz]),
    "kr_project_qkv": (i32, [vp, sz, u32, u32, u32, u32, sz]),
    "kr_project_gate_up": (i32, [vp, sz, u32, u32, u32, sz]),
    "kr_kv_write": (i32, [vp, sz, vp, u32, u32, sz]),
    "kr_attention": (i32, [vp, u32, u32, u32, sz, C.POINTER(KrWindow), sz, C.POINTER(KrAttnSpec)]),
    "kr_add_in_place": (i32, [vp, u32, u32, sz]),
    "kr_mul": (i32, [vp, u32, sz, u32, sz, u32, sz, sz]),
    "kr_conv_prefill": (i32, [vp, u32, u32, u32, sz, sz, sz]),
    "kr_conv_decode": (i32, [vp, u32, u32, u32, u32, sz, sz]),
    "kr_silu_mul": (i32, [vp, u32, u32, sz]),
    "kr_logits": (i32, [vp, u32, u32]),
    "kr_matmul": (i32, [vp, u32, u32, u32, sz]),
    "kr_matmul_noalloc": (i32, [vp, u32, u32, u32, sz]),
    "kr_matmul_noalloc_max_elems": (sz, []),
    "kr_classify": (i32, [vp, u32, u32, u32]),
    "kr_quantize_rows": (i32, [vp, u32, sz, sz]),
    "kr_matmul_quantized": (i32, [vp, u32, u32, sz]),
    "kr_matmul_quantized_set": (i32, [vp, C.POINTER(u32), C.POINTER(u32), i32, sz]),
    "kr_matmul_split": (i32, [vp, u32, u32, u32, sz]),
    "kr_stream_read": (i32, [vp, u32, sz, sz]),
    "kr_stream_read_shape": (i32, [vp, u32, sz, sz, i32, sz]),
    "kr_capture_begin": (i32, [vp]),
    "kr_capture_end": (i32, [vp]),
    "kr_replay": (i32, [vp, sz]),
    "kr_timer_start": (i32, [vp]),
    "kr_timer_stop": (i32, [vp, C.POINTER(C.c_float)]),
    "kr_dbg_quantize": (i32, [vp, u32, sz, sz, vp, vp, vp]),
    "kr_dbg_block_dots": (i32, [vp, u32, u32, sz, vp]),
    "kr_dbg_mfma_f32": (i32, [vp, vp, vp, vp, vp, sz]),
    "kr_dbg_serial_sum": (i32, [vp, vp, sz, sz, i32, vp]),
    "kr_kv_upload": (i32, [vp, i32, sz, vp, sz]),
    "kr_kv_read": (i32, [vp, i32, sz, vp, sz]),
    "kr_matrix_read": (i32, [vp, u32, vp, sz, vp, sz]),
    "kr_matrix_shape": (i32, [vp, u32, C.POINTER(sz), C.POINTER(sz), C.POINTER(i32)]),
    "kr_kv_synthetic": (i32, [vp, sz, C.c_uint64]),
    "kr_argmax": (i32, [vp, u32, sz, sz]),
    "kr_read_tokens": (i32, [vp, vp, sz]),
    "kr_synchronize": (i32, [vp]),
    "krl_llama_new": (i32, [vp, C.POINTER(KrlConfig), C.POINTER(KrlWeights), C.POINTER(vp)]),
    "krl_lfm2_new": (i32, [vp, C.POINTER(KrlConfig), C.POINTER(KrlWeights), C.POINTER(vp)]),
    "krl_free": (None, [vp]),
    "krl_last_error": (C.c_char_p, [vp]),
    "krl_forward": (i32, [vp, sz, sz, vp]),
    "krl_prefill": (i32, [vp, vp, sz, sz, vp]),
    "krl_prefill_multi": (i32, [vp, vp, vp, sz, vp]),
    "krl_prefill_shared": (i32, [vp, vp, sz, vp, vp, sz, vp]),
    "krl_decode_batch": (i32, [vp, vp, vp, vp, vp, sz, vp]),
    "krl_generate_greedy": (i32, [vp, sz, sz, sz, vp, i32]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def load() -> C.CDLL:
    """Load the in-tree library; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python kernrt_amd/build.py` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
