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

F32, BF16, F16, F64 = 0, 1, 2, 3
POLICY_AUTO, POLICY_GENERIC, POLICY_DETERMINISTIC = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.float64: F64}


def _stat_dtype(dtype):
    """Element type of LSE / delta for a storage dtype: float64 for float64, else float32."""
    return torch.float64 if dtype == torch.float64 else torch.float32

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
    lib.ctattn_fwd_workspace_bytes.argtypes = [c_int, i64, i64, i64, i64]
    lib.ctattn_fwd_workspace_bytes.restype = i64
    lib.ctattn_fwd_ws.argtypes = [c_int, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, c_int, vp]
    lib.ctattn_fwd_ws.restype = c_int
    lib.ctattn_bwd_workspace_bytes.argtypes = [c_int, i64, i64, i64, i64, c_int]
    lib.ctattn_bwd_workspace_bytes.restype = i64
    lib.ctattn_bwd_workspace_bytes_max.argtypes = [c_int, i64, i64, i64, i64, c_int]
    lib.ctattn_bwd_workspace_bytes_max.restype = i64
    lib.ctattn_bwd.argtypes = [c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64,
                               i64, i64, i64, i64, c_int, vp]
    lib.ctattn_bwd.restype = c_int
    lib.ctattn_bwd_noalloc.argtypes = [c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                       i64, i64, i64, i64, c_int, vp]
    lib.ctattn_bwd_noalloc.restype = c_int
    lib.ctattn_last_error.argtypes = []
    lib.ctattn_last_error.restype = ctypes.c_char_p
    lib.ctattn_set_policy.argtypes = [c_int]
    lib.ctattn_set_policy.restype = c_int
    lib.ctattn_get_policy.argtypes = []
    lib.ctattn_get_policy.restype = c_int
    lib.ctattn_version.argtypes = []
    lib.ctattn_version.restype = c_int
    shape5 = [i64] * 5  # B, T, E, H, d
    lib.ctattn_qkv_proj_fwd.argtypes = [c_int] + [vp] * 10 + shape5 + [vp]
    lib.ctattn_qkv_proj_fwd.restype = c_int
    lib.ctattn_qkv_proj_bwd_workspace_bytes.argtypes = [c_int] + shape5
    lib.ctattn_qkv_proj_bwd_workspace_bytes.restype = i64
    lib.ctattn_qkv_proj_bwd.argtypes = [c_int] + [vp] * 15 + [i64] + shape5 + [vp]
    lib.ctattn_qkv_proj_bwd.restype = c_int
    lib.ctattn_out_proj_fwd.argtypes = [c_int] + [vp] * 4 + shape5 + [vp]
    lib.ctattn_out_proj_fwd.restype = c_int
    lib.ctattn_out_proj_bwd_workspace_bytes.argtypes = [c_int] + shape5
    lib.ctattn_out_proj_bwd_workspace_bytes.restype = i64
    lib.ctattn_out_proj_bwd.argtypes = [c_int] + [vp] * 7 + [i64] + shape5 + [vp]
    lib.ctattn_out_proj_bwd.restype = c_int
    lib.ctattn_sgd_update.argtypes = [c_int, vp, vp, ctypes.c_double, i64, vp]
    lib.ctattn_sgd_update.restype = c_int
    f64 = ctypes.c_double
    sigs = {
        "ctattn_linear_fwd": ([c_int] + [vp] * 4 + [i64] * 3 + [vp], c_int),
        "ctattn_linear_bwd_workspace_bytes": ([c_int] + [i64] * 3, i64),
        "ctattn_linear_bwd": ([c_int] + [vp] * 7 + [i64] * 4 + [vp], c_int),
        "ctattn_linear_act_fwd": ([c_int, c_int] + [vp] * 5 + [i64] * 3 + [vp], c_int),
        "ctattn_linear_act_bwd": ([c_int, c_int] + [vp] * 8 + [i64] * 4 + [vp], c_int),
        "ctattn_layernorm_fwd": ([c_int] + [vp] * 6 + [i64, i64, f64, vp], c_int),
        "ctattn_layernorm_bwd_workspace_bytes": ([c_int, i64, i64], i64),
        "ctattn_layernorm_bwd": ([c_int] + [vp] * 9 + [i64] * 3 + [vp], c_int),
        "ctattn_activation_fwd": ([c_int, c_int, vp, vp, i64, vp], c_int),
        "ctattn_activation_bwd": ([c_int, c_int, vp, vp, vp, i64, vp], c_int),
        "ctattn_embedding_fwd": ([c_int] + [vp] * 4 + [i64] * 5 + [vp], c_int),
        "ctattn_embedding_bwd": ([c_int] + [vp] * 4 + [i64] * 4 + [vp], c_int),
        "ctattn_softmax_fwd": ([c_int, vp, vp, i64, i64, f64, vp], c_int),
        "ctattn_softmax_bwd": ([c_int, vp, vp, vp, i64, i64, f64, vp], c_int),
        "ctattn_cross_entropy_fwd": ([c_int, vp, vp, vp, i64, i64, vp], c_int),
        "ctattn_cross_entropy_bwd": ([c_int, vp, vp, vp, i64, i64, vp], c_int),
        "ctattn_softmax_cross_entropy_bwd": ([c_int, vp, vp, vp, i64, i64, f64, vp], c_int),
        "ctattn_mse_loss_fwd": ([c_int, vp, vp, vp, i64, i64, vp], c_int),
        "ctattn_mse_loss_bwd": ([c_int, vp, vp, vp, i64, i64, vp], c_int),
        "ctattn_adam_update": ([c_int, vp, vp, vp, vp, i64] + [f64] * 5 + [i64, c_int, vp], c_int),
        "ctattn_adam_update_multi": ([c_int, c_int] + [vp] * 5 + [f64] * 5 + [i64, c_int, vp], c_int),
        "ctattn_zero_multi": ([c_int, vp, vp, vp], c_int),
        "ctattn_tensor_cast": ([c_int, vp, c_int, vp, i64, vp], c_int),
        "ctattn_tensor_binary": ([c_int, c_int, vp, c_int, vp, vp, c_int, vp, vp, vp], c_int),
        "ctattn_tensor_scalar": ([c_int, c_int, vp, f64, c_int, vp, i64, vp], c_int),
        "ctattn_tensor_unary": ([c_int, c_int, vp, vp, i64, vp], c_int),
        "ctattn_tensor_reduce_workspace_bytes": ([c_int, i64, i64, i64], i64),
        "ctattn_tensor_reduce": ([c_int, c_int, vp, i64, i64, i64, vp, vp, i64, vp], c_int),
        "ctattn_tensor_permute": ([c_int, vp, c_int, vp, vp, vp, vp], c_int),
        "ctattn_tensor_kron": ([c_int, vp, vp, c_int, vp, vp, vp, vp], c_int),
        "ctattn_tensor_matmul": ([c_int, vp, vp, vp] + [i64] * 5 + [vp], c_int),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
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
        raise ValueError(f"{name}: dtype {ref.dtype} unsupported (float32, bfloat16, float16, float64)")
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
    stat = _stat_dtype(q.dtype)
    if lse is None:
        lse = torch.empty((b, h, t), dtype=stat, device=q.device)
    _check_qkv("flash_attn_fwd", q, out)
    if lse.dtype != stat or tuple(lse.shape) != (b, h, t) or not lse.is_contiguous():
        raise ValueError(f"flash_attn_fwd: lse must be contiguous {stat} [B, H, T]")
    lib = load()
    code = _DTYPE_CODE[q.dtype]
    need = lib.ctattn_fwd_workspace_bytes(code, b, h, t, d)
    if need < 0:
        raise RuntimeError(f"ctattn_fwd_workspace_bytes failed: {last_error()}")
    ws = torch.empty(need, dtype=torch.uint8, device=q.device) if need > 0 else None
    rc = lib.ctattn_fwd_ws(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                           _ptr(ws), need, b, h, t, d, int(bool(causal)), _stream_handle(stream))
    _check(rc, "ctattn_fwd_ws")
    return out, lse


def bwd_workspace_bytes(dtype, b, h, t, d, causal, fastest: bool = False) -> int:
    """ctattn_bwd_workspace_bytes (linear in B*H*T), or with fastest=True
    ctattn_bwd_workspace_bytes_max (with the dS tiles where the kernels take them: bf16 / fp16
    at d = 128, fp32 at d in {64, 128} under DETERMINISTIC and at d = 128 on large grids under
    AUTO; about B*H*T^2 bytes at 16-bit, twice that at fp32)."""
    code = _DTYPE_CODE[dtype] if isinstance(dtype, torch.dtype) else int(dtype)
    fn = "ctattn_bwd_workspace_bytes_max" if fastest else "ctattn_bwd_workspace_bytes"
    n = getattr(load(), fn)(code, b, h, t, d, int(bool(causal)))
    if n < 0:
        raise RuntimeError(f"{fn} failed: {last_error()}")
    return n


def flash_attn_bwd(q, k, v, o, do, lse, causal: bool = False, dq=None, dk=None, dv=None,
                   workspace=None, stream=None):
    """dQ, dK, dV of attention given the forward's O and LSE and the upstream dO.  Without a
    workspace one of ctattn_bwd_workspace_bytes is allocated here; a larger one (up to
    bwd_workspace_bytes(..., fastest=True)) lets the bf16 / fp16 d = 128 path store dS."""
    _check_qkv("flash_attn_bwd", q, k, v, o, do)
    b, h, t, d = q.shape
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(q) if dk is None else dk
    dv = torch.empty_like(q) if dv is None else dv
    _check_qkv("flash_attn_bwd", q, dq, dk, dv)
    stat = _stat_dtype(q.dtype)
    if lse.dtype != stat or tuple(lse.shape) != (b, h, t) or not lse.is_contiguous():
        raise ValueError(f"flash_attn_bwd: lse must be contiguous {stat} [B, H, T]")
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


NOALLOC_SCRATCH_BYTES = 32 << 20  # CTATTN_NOALLOC_SCRATCH_BYTES


def flash_attn_bwd_noalloc(q, k, v, o, do, lse, causal: bool = False, dq=None, dk=None, dv=None,
                           stream=None):
    """flash_attn_bwd through ctattn_bwd_noalloc: no workspace, the library's static scratch.
    dq / dk / dv are allocated here by torch when not given (the C entry point itself
    allocates nothing)."""
    _check_qkv("flash_attn_bwd_noalloc", q, k, v, o, do)
    b, h, t, d = q.shape
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(q) if dk is None else dk
    dv = torch.empty_like(q) if dv is None else dv
    _check_qkv("flash_attn_bwd_noalloc", q, dq, dk, dv)
    stat = _stat_dtype(q.dtype)
    if lse.dtype != stat or tuple(lse.shape) != (b, h, t) or not lse.is_contiguous():
        raise ValueError(f"flash_attn_bwd_noalloc: lse must be contiguous {stat} [B, H, T]")
    rc = load().ctattn_bwd_noalloc(_DTYPE_CODE[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   o.data_ptr(), do.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), b, h, t, d, int(bool(causal)),
                                   _stream_handle(stream))
    _check(rc, "ctattn_bwd_noalloc")
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


# ---- attention-layer projections -------------------------------------------------------


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check_dev(name, dtype, *ts):
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda or not t.is_contiguous() or t.dtype != dtype:
            raise ValueError(f"{name}: tensors must be contiguous {dtype} on the GPU")


def qkv_proj_fwd(x, wq, wk, wv, bq, bk, bv, num_heads: int, head_dim: int, stream=None):
    """Q, K, V [B, H, T, d] = x [B, T, E] W^T + b (W: [H*d, E]; biases may be None)."""
    if x.dim() != 3:
        raise ValueError("qkv_proj_fwd: x must be [B, T, E]")
    b, t, e = x.shape
    hd = num_heads * head_dim
    _check_dev("qkv_proj_fwd", x.dtype, x, wq, wk, wv, bq, bk, bv)
    for w in (wq, wk, wv):
        if tuple(w.shape) != (hd, e):
            raise ValueError(f"qkv_proj_fwd: weights must be [{hd}, {e}], got {tuple(w.shape)}")
    q, k, v = (torch.empty((b, num_heads, t, head_dim), dtype=x.dtype, device=x.device) for _ in range(3))
    rc = load().ctattn_qkv_proj_fwd(_DTYPE_CODE[x.dtype], _ptr(x), _ptr(wq), _ptr(wk), _ptr(wv), _ptr(bq),
                                    _ptr(bk), _ptr(bv), _ptr(q), _ptr(k), _ptr(v), b, t, e, num_heads,
                                    head_dim, _stream_handle(stream))
    _check(rc, "ctattn_qkv_proj_fwd")
    return q, k, v


def qkv_proj_bwd(x, dq, dk, dv, wq, wk, wv, dw=None, db=None, want_dx=True, stream=None):
    """Backward of qkv_proj_fwd.  dw / db: tuples of three tensors accumulated in place
    (or None to skip).  Returns dx [B, T, E] (or None)."""
    b, t, e = x.shape
    _, h, _, d = dq.shape
    _check_dev("qkv_proj_bwd", x.dtype, x, dq, dk, dv, wq, wk, wv, *(dw or ()), *(db or ()))
    code = _DTYPE_CODE[x.dtype]
    lib = load()
    need = lib.ctattn_qkv_proj_bwd_workspace_bytes(code, b, t, e, h, d)
    if need < 0:
        raise RuntimeError(f"ctattn_qkv_proj_bwd_workspace_bytes failed: {last_error()}")
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    dx = torch.empty_like(x) if want_dx else None
    dw = dw or (None, None, None)
    db = db or (None, None, None)
    rc = lib.ctattn_qkv_proj_bwd(code, _ptr(x), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(wq), _ptr(wk), _ptr(wv),
                                 *map(_ptr, dw), *map(_ptr, db), _ptr(dx), _ptr(ws), ws.numel(), b, t, e, h,
                                 d, _stream_handle(stream))
    _check(rc, "ctattn_qkv_proj_bwd")
    return dx


def out_proj_fwd(c, wo, bo, stream=None):
    """y [B, T, E] = c W_o^T + b_o, c: attention output [B, H, T, d], W_o: [E, H*d]."""
    b, h, t, d = c.shape
    e = wo.shape[0]
    _check_dev("out_proj_fwd", c.dtype, c, wo, bo)
    if tuple(wo.shape) != (e, h * d):
        raise ValueError(f"out_proj_fwd: wo must be [E, {h * d}]")
    y = torch.empty((b, t, e), dtype=c.dtype, device=c.device)
    rc = load().ctattn_out_proj_fwd(_DTYPE_CODE[c.dtype], _ptr(c), _ptr(wo), _ptr(bo), _ptr(y), b, t, e, h, d,
                                    _stream_handle(stream))
    _check(rc, "ctattn_out_proj_fwd")
    return y


def out_proj_bwd(c, dy, wo, dwo=None, dbo=None, want_dc=True, stream=None):
    """Backward of out_proj_fwd: dwo / dbo accumulated in place (None to skip); returns dc."""
    b, h, t, d = c.shape
    e = wo.shape[0]
    _check_dev("out_proj_bwd", c.dtype, c, dy, wo, dwo, dbo)
    code = _DTYPE_CODE[c.dtype]
    lib = load()
    need = lib.ctattn_out_proj_bwd_workspace_bytes(code, b, t, e, h, d)
    if need < 0:
        raise RuntimeError(f"ctattn_out_proj_bwd_workspace_bytes failed: {last_error()}")
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=c.device)
    dc = torch.empty_like(c) if want_dc else None
    rc = lib.ctattn_out_proj_bwd(code, _ptr(c), _ptr(dy), _ptr(wo), _ptr(dwo), _ptr(dbo), _ptr(dc), _ptr(ws),
                                 ws.numel(), b, t, e, h, d, _stream_handle(stream))
    _check(rc, "ctattn_out_proj_bwd")
    return dc


def sgd_update(params, grads, lr: float, stream=None):
    """params -= lr * grads, in place, on the GPU."""
    _check_dev("sgd_update", params.dtype, params, grads)
    if params.numel() != grads.numel():
        raise ValueError("sgd_update: size mismatch")
    rc = load().ctattn_sgd_update(_DTYPE_CODE[params.dtype], _ptr(params), _ptr(grads), float(lr),
                                  params.numel(), _stream_handle(stream))
    _check(rc, "ctattn_sgd_update")


# ---- layers around attention (NanoGPT training step) -----------------------------------

ACT_RELU, ACT_GELU, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3


def _rows(x, last: int, name: str) -> int:
    if x.dim() < 1 or x.shape[-1] != last:
        raise ValueError(f"{name}: last dimension must be {last}, got {tuple(x.shape)}")
    return x.numel() // last if last else 0


def _workspace(need: int, fn: str, device):
    if need < 0:
        raise RuntimeError(f"{fn} failed: {last_error()}")
    return torch.empty(max(need, 1), dtype=torch.uint8, device=device)


def _check_ids(name, *ts):
    for t in ts:
        if not t.is_cuda or not t.is_contiguous() or t.dtype != torch.int32:
            raise ValueError(f"{name}: ids / targets must be contiguous int32 on the GPU")


def linear_fwd(x, w, b=None, stream=None):
    """y [..., N] = x [..., K] w^T + b (w: [N, K], b: [N] or None)."""
    n, k = w.shape
    m = _rows(x, k, "linear_fwd")
    _check_dev("linear_fwd", x.dtype, x, w, b)
    y = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
    rc = load().ctattn_linear_fwd(_DTYPE_CODE[x.dtype], _ptr(x), _ptr(w), _ptr(b), _ptr(y), m, n, k,
                                  _stream_handle(stream))
    _check(rc, "ctattn_linear_fwd")
    return y


def linear_bwd(x, w, dy, dw=None, db=None, want_dx=True, stream=None):
    """dw += dy^T x, db += colsum(dy) in place (None to skip); returns dx = dy w (or None)."""
    n, k = w.shape
    m = _rows(x, k, "linear_bwd")
    if _rows(dy, n, "linear_bwd") != m:
        raise ValueError("linear_bwd: dy rows do not match x")
    _check_dev("linear_bwd", x.dtype, x, w, dy, dw, db)
    code = _DTYPE_CODE[x.dtype]
    lib = load()
    ws = _workspace(lib.ctattn_linear_bwd_workspace_bytes(code, m, n, k), "ctattn_linear_bwd_workspace_bytes",
                    x.device)
    dx = torch.empty_like(x) if want_dx else None
    rc = lib.ctattn_linear_bwd(code, _ptr(x), _ptr(w), _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db), _ptr(ws),
                               ws.numel(), m, n, k, _stream_handle(stream))
    _check(rc, "ctattn_linear_bwd")
    return dx


def linear_act_fwd(x, w, b, kind: int, stream=None):
    """(pre, y): pre = x w^T + b and y = act(pre) from one launch (ctattn_linear_act_fwd)."""
    n, k = w.shape
    m = _rows(x, k, "linear_act_fwd")
    _check_dev("linear_act_fwd", x.dtype, x, w, b)
    pre = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
    y = torch.empty_like(pre)
    rc = load().ctattn_linear_act_fwd(_DTYPE_CODE[x.dtype], int(kind), _ptr(x), _ptr(w), _ptr(b), _ptr(pre), _ptr(y),
                                      m, n, k, _stream_handle(stream))
    _check(rc, "ctattn_linear_act_fwd")
    return pre, y


def linear_act_bwd(x, w, dy, pre, kind: int, dw=None, db=None, stream=None):
    """Backward of act then linear (x = act(pre) is the linear layer's input): dw += dy^T x,
    db += colsum(dy) in place (None to skip); returns dpre = act'(pre) * (dy w)."""
    n, k = w.shape
    m = _rows(x, k, "linear_act_bwd")
    if _rows(dy, n, "linear_act_bwd") != m or pre.shape != x.shape:
        raise ValueError("linear_act_bwd: dy / pre shapes do not match x")
    _check_dev("linear_act_bwd", x.dtype, x, w, dy, pre, dw, db)
    code = _DTYPE_CODE[x.dtype]
    lib = load()
    ws = _workspace(lib.ctattn_linear_bwd_workspace_bytes(code, m, n, k), "ctattn_linear_bwd_workspace_bytes",
                    x.device)
    dpre = torch.empty_like(x)
    rc = lib.ctattn_linear_act_bwd(code, int(kind), _ptr(x), _ptr(w), _ptr(dy), _ptr(pre), _ptr(dpre), _ptr(dw),
                                   _ptr(db), _ptr(ws), ws.numel(), m, n, k, _stream_handle(stream))
    _check(rc, "ctattn_linear_act_bwd")
    return dpre


def layernorm_fwd(x, gamma, beta, eps: float = 1e-5, stream=None):
    """Returns (y, mean, rstd): LayerNorm over the last dimension; the row statistics are
    float64 for float64 input, float32 otherwise."""
    d = gamma.numel()
    n = _rows(x, d, "layernorm_fwd")
    _check_dev("layernorm_fwd", x.dtype, x, gamma, beta)
    y = torch.empty_like(x)
    mean = torch.empty(n, dtype=_stat_dtype(x.dtype), device=x.device)
    rstd = torch.empty(n, dtype=_stat_dtype(x.dtype), device=x.device)
    rc = load().ctattn_layernorm_fwd(_DTYPE_CODE[x.dtype], _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), _ptr(mean),
                                     _ptr(rstd), n, d, float(eps), _stream_handle(stream))
    _check(rc, "ctattn_layernorm_fwd")
    return y, mean, rstd


def layernorm_bwd(x, gamma, dy, mean, rstd, dgamma=None, dbeta=None, stream=None):
    """Returns dx; dgamma / dbeta accumulated in place (None to skip)."""
    d = gamma.numel()
    n = _rows(x, d, "layernorm_bwd")
    _check_dev("layernorm_bwd", x.dtype, x, gamma, dy, dgamma, dbeta)
    _check_dev("layernorm_bwd", _stat_dtype(x.dtype), mean, rstd)
    code = _DTYPE_CODE[x.dtype]
    lib = load()
    ws = _workspace(lib.ctattn_layernorm_bwd_workspace_bytes(code, n, d), "ctattn_layernorm_bwd_workspace_bytes",
                    x.device)
    dx = torch.empty_like(x)
    rc = lib.ctattn_layernorm_bwd(code, _ptr(x), _ptr(gamma), _ptr(dy), _ptr(mean), _ptr(rstd), _ptr(dx),
                                  _ptr(dgamma), _ptr(dbeta), _ptr(ws), ws.numel(), n, d, _stream_handle(stream))
    _check(rc, "ctattn_layernorm_bwd")
    return dx


def activation_fwd(x, kind: int, stream=None):
    _check_dev("activation_fwd", x.dtype, x)
    y = torch.empty_like(x)
    rc = load().ctattn_activation_fwd(_DTYPE_CODE[x.dtype], int(kind), _ptr(x), _ptr(y), x.numel(),
                                      _stream_handle(stream))
    _check(rc, "ctattn_activation_fwd")
    return y


def activation_bwd(x, dy, kind: int, stream=None):
    _check_dev("activation_bwd", x.dtype, x, dy)
    dx = torch.empty_like(x)
    rc = load().ctattn_activation_bwd(_DTYPE_CODE[x.dtype], int(kind), _ptr(x), _ptr(dy), _ptr(dx), x.numel(),
                                      _stream_handle(stream))
    _check(rc, "ctattn_activation_bwd")
    return dx


def embedding_fwd(ids, tok=None, pos=None, stream=None):
    """out [B, T, E] = tok[ids] + pos[t] (either table may be None); ids int32 [B, T]."""
    table = tok if tok is not None else pos
    b, t = ids.shape
    e = table.shape[1]
    _check_ids("embedding_fwd", ids)
    _check_dev("embedding_fwd", table.dtype, tok, pos)
    vocab = tok.shape[0] if tok is not None else 1
    max_len = pos.shape[0] if pos is not None else max(t, 1)
    out = torch.empty((b, t, e), dtype=table.dtype, device=ids.device)
    rc = load().ctattn_embedding_fwd(_DTYPE_CODE[table.dtype], _ptr(ids), _ptr(tok), _ptr(pos), _ptr(out), b, t, e,
                                     vocab, max_len, _stream_handle(stream))
    _check(rc, "ctattn_embedding_fwd")
    return out


def embedding_bwd(ids, dout, dtok=None, dpos=None, vocab: int | None = None, stream=None):
    """dtok[ids] += dout, dpos[t] += sum_b dout (in place, dout's dtype; either may be None)."""
    b, t = ids.shape
    e = dout.shape[-1]
    _check_ids("embedding_bwd", ids)
    _check_dev("embedding_bwd", dout.dtype, dout, dtok, dpos)
    vocab = vocab if vocab is not None else (dtok.shape[0] if dtok is not None else 1)
    rc = load().ctattn_embedding_bwd(_DTYPE_CODE[dout.dtype], _ptr(ids), _ptr(dout), _ptr(dtok), _ptr(dpos), b, t, e, vocab,
                                     _stream_handle(stream))
    _check(rc, "ctattn_embedding_bwd")


def softmax_fwd(z, temperature: float = 1.0, stream=None):
    v = z.shape[-1]
    _check_dev("softmax_fwd", z.dtype, z)
    p = torch.empty_like(z)
    rc = load().ctattn_softmax_fwd(_DTYPE_CODE[z.dtype], _ptr(z), _ptr(p), _rows(z, v, "softmax_fwd"), v,
                                   float(temperature), _stream_handle(stream))
    _check(rc, "ctattn_softmax_fwd")
    return p


def softmax_bwd(p, dp, temperature: float = 1.0, stream=None):
    v = p.shape[-1]
    _check_dev("softmax_bwd", p.dtype, p, dp)
    dz = torch.empty_like(p)
    rc = load().ctattn_softmax_bwd(_DTYPE_CODE[p.dtype], _ptr(p), _ptr(dp), _ptr(dz), _rows(p, v, "softmax_bwd"), v,
                                   float(temperature), _stream_handle(stream))
    _check(rc, "ctattn_softmax_bwd")
    return dz


def cross_entropy_fwd(p, target, stream=None):
    """Per-row -log p[target] / N (the shape of target; float64 for float64 p, else float32)."""
    v = p.shape[-1]
    n = _rows(p, v, "cross_entropy_fwd")
    _check_dev("cross_entropy_fwd", p.dtype, p)
    _check_ids("cross_entropy_fwd", target)
    if target.numel() != n:
        raise ValueError("cross_entropy_fwd: one target per row")
    loss = torch.empty(target.shape, dtype=_stat_dtype(p.dtype), device=p.device)
    rc = load().ctattn_cross_entropy_fwd(_DTYPE_CODE[p.dtype], _ptr(p), _ptr(target), _ptr(loss), n, v,
                                         _stream_handle(stream))
    _check(rc, "ctattn_cross_entropy_fwd")
    return loss


def cross_entropy_bwd(p, target, stream=None):
    v = p.shape[-1]
    n = _rows(p, v, "cross_entropy_bwd")
    _check_dev("cross_entropy_bwd", p.dtype, p)
    _check_ids("cross_entropy_bwd", target)
    dp = torch.empty_like(p)
    rc = load().ctattn_cross_entropy_bwd(_DTYPE_CODE[p.dtype], _ptr(p), _ptr(target), _ptr(dp), n, v,
                                         _stream_handle(stream))
    _check(rc, "ctattn_cross_entropy_bwd")
    return dp


def softmax_cross_entropy_bwd(p, target, temperature: float = 1.0, stream=None):
    v = p.shape[-1]
    n = _rows(p, v, "softmax_cross_entropy_bwd")
    _check_dev("softmax_cross_entropy_bwd", p.dtype, p)
    _check_ids("softmax_cross_entropy_bwd", target)
    dz = torch.empty_like(p)
    rc = load().ctattn_softmax_cross_entropy_bwd(_DTYPE_CODE[p.dtype], _ptr(p), _ptr(target), _ptr(dz), n, v,
                                                 float(temperature), _stream_handle(stream))
    _check(rc, "ctattn_softmax_cross_entropy_bwd")
    return dz


def mse_loss_fwd(x, target, stream=None):
    """Per-row mean of (x - target)^2 over the last dimension (float64 for float64 x, else
    float32; the shape of x without its last dimension)."""
    d = x.shape[-1]
    n = _rows(x, d, "mse_loss_fwd")
    _check_dev("mse_loss_fwd", x.dtype, x, target)
    if target.shape != x.shape:
        raise ValueError("mse_loss_fwd: x and target shapes differ")
    loss = torch.empty(x.shape[:-1], dtype=_stat_dtype(x.dtype), device=x.device)
    rc = load().ctattn_mse_loss_fwd(_DTYPE_CODE[x.dtype], _ptr(x), _ptr(target), _ptr(loss), n, d,
                                    _stream_handle(stream))
    _check(rc, "ctattn_mse_loss_fwd")
    return loss


def mse_loss_bwd(x, target, stream=None):
    d = x.shape[-1]
    n = _rows(x, d, "mse_loss_bwd")
    _check_dev("mse_loss_bwd", x.dtype, x, target)
    if target.shape != x.shape:
        raise ValueError("mse_loss_bwd: x and target shapes differ")
    dx = torch.empty_like(x)
    rc = load().ctattn_mse_loss_bwd(_DTYPE_CODE[x.dtype], _ptr(x), _ptr(target), _ptr(dx), n, d,
                                    _stream_handle(stream))
    _check(rc, "ctattn_mse_loss_bwd")
    return dx


def adam_update(param, grad, m, v, step: int, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
                decoupled: bool = False, stream=None):
    """One Adam (decoupled=False) or AdamW step, in place on param / m / v (moments float64 for
    float64 parameters, float32 otherwise)."""
    _check_dev("adam_update", param.dtype, param, grad)
    _check_dev("adam_update", _stat_dtype(param.dtype), m, v)
    n = param.numel()
    if not (grad.numel() == m.numel() == v.numel() == n):
        raise ValueError("adam_update: size mismatch")
    rc = load().ctattn_adam_update(_DTYPE_CODE[param.dtype], _ptr(param), _ptr(grad), _ptr(m), _ptr(v), n, float(lr), float(beta1),
                                   float(beta2), float(eps), float(weight_decay), int(step), int(bool(decoupled)),
                                   _stream_handle(stream))
    _check(rc, "ctattn_adam_update")


def _ptr_table(ts):
    arr = (ctypes.c_void_p * max(len(ts), 1))()
    for i, t in enumerate(ts):
        arr[i] = None if t is None else t.data_ptr()
    return arr


def adam_update_multi(params, grads, ms, vs, step: int, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                      weight_decay=0.0, decoupled: bool = False, stream=None):
    """ctattn_adam_update over lists of tensors of one dtype, one launch per 32 tensors."""
    if not (len(params) == len(grads) == len(ms) == len(vs)):
        raise ValueError("adam_update_multi: list lengths differ")
    dtype = params[0].dtype if params else torch.float32
    for p, g, m, v in zip(params, grads, ms, vs):
        _check_dev("adam_update_multi", dtype, p, g)
        _check_dev("adam_update_multi", _stat_dtype(dtype), m, v)
        if len({t.numel() for t in (p, g, m, v)}) != 1:
            raise ValueError("adam_update_multi: size mismatch")
    n = (ctypes.c_int64 * max(len(params), 1))(*[p.numel() for p in params])
    rc = load().ctattn_adam_update_multi(_DTYPE_CODE[dtype], len(params), _ptr_table(params), _ptr_table(grads), _ptr_table(ms),
                                         _ptr_table(vs), n, float(lr), float(beta1), float(beta2), float(eps),
                                         float(weight_decay), int(step), int(bool(decoupled)), _stream_handle(stream))
    _check(rc, "ctattn_adam_update_multi")


def zero_multi(tensors, stream=None):
    """Zeroes a list of device tensors in one launch per 32 tensors."""
    for t in tensors:
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("zero_multi: tensors must be contiguous on the GPU")
    nb = (ctypes.c_int64 * max(len(tensors), 1))(*[t.numel() * t.element_size() for t in tensors])
    rc = load().ctattn_zero_multi(len(tensors), _ptr_table(tensors), nb, _stream_handle(stream))
    _check(rc, "ctattn_zero_multi")
