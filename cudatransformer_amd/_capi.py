"""ctypes binding of libctattn.so (the C-ABI in include/ctattn.h) over torch device tensors.

torch supplies device memory and the stream (``torch.cuda.current_stream()``); every
computation runs in the HIP kernels of libctattn.so.  There is no CPU or torch fallback:
if the library is missing or a call fails, a RuntimeError is raised.

``import torch`` must happen before libctattn.so is loaded so that the library binds to
the HIP runtime torch already loaded (both carry the soname libamdhip64.so.7); this module
imports torch first for that reason.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libctattn.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "ctattn.h")

F32, BF16 = 0, 1
POLICY_AUTO, POLICY_GENERIC, POLICY_DETERMINISTIC = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16}

_lib = None


def header_functions() -> list[str]:
    """Names of the functions include/ctattn.h declares."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(ctattn_\w+)\s*\(", text)


def load() -> ctypes.CDLL:
    """Loads libctattn.so once and declares every C-ABI signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            " or `make -C cudatransformer_amd/csrc`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.ctattn_fwd.argtypes = [c_int, vp, vp, vp, vp, vp, i64, i64, i64, i64, c_int, vp]
    lib.ctattn_fwd.restype = c_int
    lib.ctattn_bwd_workspace_bytes.argtypes = [c_int, i64, i64, i64, i64, c_int]
    lib.ctattn_bwd_workspace_bytes.restype = i64
    lib.ctattn_bwd.argtypes = [c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64,
                               i64, i64, i64, i64, c_int, vp]
    lib.ctattn_bwd.restype = c_int
    lib.ctattn_last_error.argtypes = []
    lib.ctattn_last_error.restype = ctypes.c_char_p
    lib.ctattn_set_policy.argtypes = [c_int]
    lib.ctattn_set_policy.restype = c_int
    lib.ctattn_get_policy.argtypes = []
    lib.ctattn_get_policy.restype = c_int
    lib.ctattn_version.argtypes = []
    lib.ctattn_version.restype = c_int
    _lib = lib
    return lib


def last_error() -> str:
    return load().ctattn_last_error().decode()


def _check(rc: int, fn: str):
    if rc != 0:
        raise RuntimeError(f"{fn} failed with hipError {rc}: {last_error()}")


def set_policy(policy: int) -> int:
    prev = load().ctattn_set_policy(int(policy))
    if prev < 0:
        raise ValueError(f"unknown policy {policy}")
    return prev


def _stream_handle(stream) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _check_qkv(name, *ts):
    ref = ts[0]
    if ref.dim() != 4:
        raise ValueError(f"{name}: tensors must be [B, H, T, d], got {tuple(ref.shape)}")
    if ref.dtype not in _DTYPE_CODE:
        raise ValueError(f"{name}: dtype {ref.dtype} unsupported (float32 or bfloat16)")
    for t in ts:
        if not t.is_cuda:
            raise ValueError(f"{name}: tensors must live on the GPU")
        if t.shape != ref.shape or t.dtype != ref.dtype:
            raise ValueError(f"{name}: shape/dtype mismatch {tuple(t.shape)} {t.dtype} vs "
                             f"{tuple(ref.shape)} {ref.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{name}: tensors must be contiguous")


def flash_attn_fwd(q, k, v, causal: bool = False, out=None, lse=None, stream=None):
    """O, LSE = attention(q, k, v); q, k, v contiguous [B, H, T, d] on the GPU."""
    _check_qkv("flash_attn_fwd", q, k, v)
    b, h, t, d = q.shape
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty((b, h, t), dtype=torch.float32, device=q.device)
    _check_qkv("flash_attn_fwd", q, out)
    if lse.dtype != torch.float32 or tuple(lse.shape) != (b, h, t) or not lse.is_contiguous():
        raise ValueError("flash_attn_fwd: lse must be contiguous float32 [B, H, T]")
    rc = load().ctattn_fwd(_DTYPE_CODE[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           out.data_ptr(), lse.data_ptr(), b, h, t, d, int(bool(causal)),
                           _stream_handle(stream))
    _check(rc, "ctattn_fwd")
    return out, lse


def bwd_workspace_bytes(dtype, b, h, t, d, causal) -> int:
    code = _DTYPE_CODE[dtype] if isinstance(dtype, torch.dtype) else int(dtype)
    n = load().ctattn_bwd_workspace_bytes(code, b, h, t, d, int(bool(causal)))
    if n < 0:
        raise RuntimeError(f"ctattn_bwd_workspace_bytes failed: {last_error()}")
    return n


def flash_attn_bwd(q, k, v, o, do, lse, causal: bool = False, dq=None, dk=None, dv=None,
                   workspace=None, stream=None):
    """dQ, dK, dV of attention given the forward's O and LSE and the upstream dO."""
    _check_qkv("flash_attn_bwd", q, k, v, o, do)
    b, h, t, d = q.shape
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(q) if dk is None else dk
    dv = torch.empty_like(q) if dv is None else dv
    _check_qkv("flash_attn_bwd", q, dq, dk, dv)
    if lse.dtype != torch.float32 or tuple(lse.shape) != (b, h, t) or not lse.is_contiguous():
        raise ValueError("flash_attn_bwd: lse must be contiguous float32 [B, H, T]")
    need = bwd_workspace_bytes(q.dtype, b, h, t, d, causal)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"flash_attn_bwd: workspace too small ({need} bytes needed)")
    rc = load().ctattn_bwd(_DTYPE_CODE[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           o.data_ptr(), do.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                           dk.data_ptr(), dv.data_ptr(), workspace.data_ptr(),
                           workspace.numel() * workspace.element_size(), b, h, t, d,
                           int(bool(causal)), _stream_handle(stream))
    _check(rc, "ctattn_bwd")
    return dq, dk, dv


class FlashAttentionFunction(torch.autograd.Function):
    """torch.autograd wrapper: forward/backward both run the ctattn kernels."""

    @staticmethod
    def forward(ctx, q, k, v, causal=False):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        o, lse = flash_attn_fwd(q, k, v, causal)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.causal = causal
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = flash_attn_bwd(q, k, v, o, do.contiguous(), lse, ctx.causal)
        return dq, dk, dv, None


def flash_attention(q, k, v, causal: bool = False):
    """Differentiable attention on the ctattn kernels."""
    return FlashAttentionFunction.apply(q, k, v, causal)
