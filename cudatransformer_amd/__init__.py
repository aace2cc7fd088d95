"""MI355X-native flash attention for the CudaTransformer FlashAttentionLayer path.

Layers of this package
  * ``libctattn.so``   -- HIP kernels for gfx950 behind a C-ABI (``include/ctattn.h``).
  * ``cuda_transformer`` -- C++ host module (pybind11) mirroring the reference's
    ``Tensor`` / ``FlashAttentionLayer`` API on top of that C-ABI.
  * ``_capi``          -- ctypes binding of the same C-ABI over torch device tensors
    (torch is plumbing: memory and streams).

torch is imported first so every native library here binds to the HIP runtime torch
loaded (one runtime per process).
"""
import torch  # noqa: F401  (must precede loading the native libraries)

from ._capi import (  # noqa: E402
    BF16,
    F32,
    POLICY_AUTO,
    POLICY_DETERMINISTIC,
    POLICY_GENERIC,
    FlashAttentionFunction,
    bwd_workspace_bytes,
    flash_attention,
    flash_attn_bwd,
    flash_attn_fwd,
    last_error,
    out_proj_bwd,
    out_proj_fwd,
    qkv_proj_bwd,
    qkv_proj_fwd,
    set_policy,
    sgd_update,
)

__all__ = [
    "BF16",
    "F32",
    "POLICY_AUTO",
    "POLICY_DETERMINISTIC",
    "POLICY_GENERIC",
    "FlashAttentionFunction",
    "bwd_workspace_bytes",
    "flash_attention",
    "flash_attn_bwd",
    "flash_attn_fwd",
    "out_proj_bwd",
    "out_proj_fwd",
    "qkv_proj_bwd",
    "qkv_proj_fwd",
    "sgd_update",
    "last_error",
    "set_policy",
]
