"""Dense fp64 restatement of scaled-dot-product attention, forward and backward.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference algorithm (``/root/reference/cuda_transformer``):

* forward, ``flash_attention.cu:57-169``: per (batch, head) the score of query row i
  against key row j is ``Q_i . K_j / sqrt(d)`` -- a *division* by sqrt(headDim)
  (``flash_attention.cu:113-116``).  The online softmax (``:120-141``) yields the row
  max ``m_i`` and denominator ``l_i``; ``O_i = sum_j exp(S_ij - m_i) V_j / l_i``
  (``:142-161``).  ``m`` and ``l`` are saved for the backward (``:164-167``); this
  build saves the single logsumexp ``LSE_i = m_i + ln l_i`` instead.
* backward, ``flash_attention.cu:226-326``: ``P_ij = exp(S_ij - m_i) / l_i``
  (``:297-298``), ``delta_i = O_i . dO_i`` (``:269-273``),
  ``dS_ij = P_ij (dO_i . V_j - delta_i) / sqrt(d)`` (``:299``), ``dQ_i = sum_j dS_ij K_j``
  (``:311``).  The reference's dK / dV loops (``:312-313, :319-321``) sum over the wrong
  index; this restatement uses the gradient of the forward instead:
  ``dK_j = sum_i dS_ij Q_i`` and ``dV_j = sum_i P_ij dO_i``.

Departures from the reference, all deliberate:

* ``causal=True`` masks ``j > i`` to ``-inf`` (the reference has no mask at all).
* keys past the sequence end do not exist (the reference zero-pads them to score 0
  when ``T % 32 != 0``, ``flash_attention.cu:104-117``).
* everything is fp64, after first rounding the inputs to the run's storage dtype
  (``cast_inputs``), so the golden reflects exactly what the kernel was given.

Layout: every tensor is ``[B, H, T, d]`` (row-major), ``lse`` is ``[B, H, T]``; this is the
layout ``attention_qkv_kernels.cu:112-120`` writes and ``attention_proj_kernels.cu:72-77``
reads.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "round_to_bf16",
    "round_to_f16",
    "cast_inputs",
    "scores",
    "attention_fwd",
    "attention_bwd",
    "attention_fwd_bwd",
    "make_inputs",
]


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bfloat16 (ties to even); returns float32.

    bfloat16 is the upper 16 bits of an IEEE binary32; rounding adds
    ``0x7FFF + lsb`` to the 32-bit pattern before truncating the low half.
    NaN/Inf are not expected in attention inputs and are not special-cased.
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = ((u + 0x7FFF + lsb) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def round_to_f16(x: np.ndarray) -> np.ndarray:
    """Round to the nearest IEEE binary16 (numpy's float16 cast, ties to even); returns
    float32."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float32)


def cast_inputs(arrays, dtype: str):
    """Round each array to the storage dtype ("f32", "bf16", "f16" or "f64") and promote to
    fp64."""
    out = []
    for a in arrays:
        if dtype == "f32":
            out.append(np.asarray(a, dtype=np.float32).astype(np.float64))
        elif dtype == "bf16":
            out.append(round_to_bf16(a).astype(np.float64))
        elif dtype == "f16":
            out.append(round_to_f16(a).astype(np.float64))
        elif dtype == "f64":
            out.append(np.asarray(a, dtype=np.float64))
        else:
            raise ValueError(f"unknown dtype {dtype!r}")
    return out


def _check_shapes(q, k, v):
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must share one [B,H,T,d] shape, got {q.shape}, {k.shape}, {v.shape}")


def scores(q: np.ndarray, k: np.ndarray, causal: bool) -> np.ndarray:
    """S = Q K^T / sqrt(d), with -inf above the diagonal when causal.

    Division by sqrt(d) as in ``flash_attention.cu:116``.
    """
    d = q.shape[-1]
    s = np.matmul(q, np.swapaxes(k, -1, -2)) / np.sqrt(np.float64(d))
    if causal:
        t = q.shape[-2]
        mask = np.triu(np.ones((t, t), dtype=bool), k=1)
        s = np.where(mask, -np.inf, s)
    return s


def attention_fwd(q, k, v, causal: bool = False):
    """Forward pass in fp64. Returns ``(O [B,H,T,d], LSE [B,H,T])``.

    ``flash_attention.cu:97-161``: running max / denominator over key tiles; the dense
    form below is the same quantity (max over all keys, sum of exp(S - m)).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    _check_shapes(q, k, v)
    s = scores(q, k, causal)
    m = s.max(axis=-1)
    p = np.exp(s - m[..., None])
    l = p.sum(axis=-1)
    o = np.matmul(p, v) / l[..., None]
    lse = m + np.log(l)
    return o, lse


def attention_bwd(q, k, v, o, do, lse, causal: bool = False):
    """Backward pass in fp64. Returns ``(dQ, dK, dV)``.

    ``flash_attention.cu:269-273`` (delta), ``:297-299`` (P, dS), ``:311`` (dQ); dK, dV from
    the gradient of the forward (not the reference's defective ``:312-313``).
    """
    q, k, v, o, do = (np.asarray(a, dtype=np.float64) for a in (q, k, v, o, do))
    lse = np.asarray(lse, dtype=np.float64)
    _check_shapes(q, k, v)
    d = q.shape[-1]
    sqrt_d = np.sqrt(np.float64(d))
    s = scores(q, k, causal)
    p = np.exp(s - lse[..., None])
    dv = np.matmul(np.swapaxes(p, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(v, -1, -2))
    delta = np.sum(do * o, axis=-1)
    ds = p * (dp - delta[..., None])
    dq = np.matmul(ds, k) / sqrt_d
    dk = np.matmul(np.swapaxes(ds, -1, -2), q) / sqrt_d
    return dq, dk, dv


def attention_fwd_bwd(q, k, v, do, causal: bool = False, chunk_heads: int = 8):
    """Forward + backward, evaluated a few (b, h) slices at a time to bound memory.

    Returns a dict with ``o, lse, dq, dk, dv`` (fp64).  ``chunk_heads`` bounds the
    number of [T, T] score matrices alive at once.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    _check_shapes(q, k, v)
    b, h, t, d = q.shape
    flat = lambda a: a.reshape(b * h, 1, t, d)  # noqa: E731
    qf, kf, vf, dof = flat(q), flat(k), flat(v), flat(do)
    o = np.empty((b * h, 1, t, d))
    lse = np.empty((b * h, 1, t))
    dq = np.empty_like(o)
    dk = np.empty_like(o)
    dv = np.empty_like(o)
    for i in range(0, b * h, chunk_heads):
        sl = slice(i, i + chunk_heads)
        o[sl], lse[sl] = attention_fwd(qf[sl], kf[sl], vf[sl], causal)
        dq[sl], dk[sl], dv[sl] = attention_bwd(qf[sl], kf[sl], vf[sl], o[sl], dof[sl], lse[sl], causal)
    shape4 = (b, h, t, d)
    return {
        "o": o.reshape(shape4),
        "lse": lse.reshape(b, h, t),
        "dq": dq.reshape(shape4),
        "dk": dk.reshape(shape4),
        "dv": dv.reshape(shape4),
    }


def make_inputs(shape, seed: int, std: float = 1.0, dtype: str = "f32"):
    """Synthetic inputs: draw Q, K, V, dO in that order from ``default_rng(seed)`` in fp64,
    scale by ``std`` and round to the storage dtype.  Returns float32 arrays (bf16 and f16
    values are returned as float32 holding exactly-representable numbers), or float64 arrays
    for dtype "f64"."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(4):
        a = rng.standard_normal(size=shape) * std
        if dtype == "bf16":
            out.append(round_to_bf16(a))
        elif dtype == "f16":
            out.append(round_to_f16(a))
        elif dtype == "f64":
            out.append(a)
        else:
            out.append(a.astype(np.float32))
    return out
