"""kernrt_amd: an MI355X (gfx950) HIP backend for KernRT's Q8_0/Q8_0x4 path.

The compute lives in libkernrt_hip.so (hand-written HIP kernels behind the C
ABI in include/kernrt_hip.h); this package is the thin host mirror of the
reference's backend seam (`backends`), model drivers (`llm`) and checkpoint
loaders (`safetensors`, `hf`).
"""

from .backends import (AttnSpec, BackendError, Hip, KvSpec, LayerWeights, ModelWeights, Q8Matrix,
                       RopeSpec, SourceMatrix, Window, available, from_env, open)
from .llm import Config, Model
from . import hf, safetensors

__all__ = ["AttnSpec", "BackendError", "Config", "Hip", "KvSpec", "LayerWeights", "Model", "ModelWeights",
           "Q8Matrix", "RopeSpec", "SourceMatrix", "Window", "available", "from_env", "hf", "open", "safetensors"]
