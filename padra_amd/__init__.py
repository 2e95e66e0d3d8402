"""padra_amd -- MI355X (gfx950) kernels for Padra's exact-fusions-v1 per-token layer path.

Host-side mirror of the reference's kernel interface for this path, over the C-ABI
declared in include/padra_hip.h (libpadra_hip.so, built in-tree by padra_amd/build.py).
The reference launches the same operations from RunCudaInferenceCore
(/root/reference/src/cuda/inference.cu:2988-3166 decode, :3421-3950 prefill).

Device memory and streams come from PyTorch (ROCm build); every operation runs in the
HIP library.  There is no CPU fallback: if the library is missing, importing the ops
raises.
"""
from __future__ import annotations

import ctypes
import os

from .abi import (  # noqa: F401
    ACT_BF16,
    ACT_F32,
    KV_BF16,
    KV_Q8,
    KV_Q8_0,
    KV_Q8_0_NOROT,
    POS_BASE,
    POS_DECODE,
    POS_PREFILL,
    TREE_128,
    TREE_256,
    DecodeState,
    KVCache,
    PadraError,
    Positions,
    PrefillState,
    lib,
    library_path,
)
from .ops import (  # noqa: F401
    Combine,
    CombineNorm,
    DecodeAttention,
    Embed,
    KVCheckpointCapture,
    KVCommit,
    KVStore,
    KvQ8_0Dequantize,
    KvQ8_0DequantizePrefix,
    NormFP8,
    QuantizeFP8,
    ResidualNormQKRopeStore,
    ResidualPostNorm,
    QKNormRopeStore,
    RopeTable,
    RotateRows,
    SiluTableBuild,
    SwiGLU,
    kv_cache,
    kv_cache_layout,
    positions_base,
    positions_decode,
    positions_prefill,
    q8_0_row_bytes,
)

__all__ = [name for name in dir() if not name.startswith("_")]
