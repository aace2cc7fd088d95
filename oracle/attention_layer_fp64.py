"""Dense fp64 restatement of the attention layer: QKV projection -> attention -> output
projection, forward and backward.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference algorithm (``/root/reference/cuda_transformer``):

* ``AttentionLayer::forward`` (``AttentionLayer.cu:75-102``): QKV projection, attention
  core, output projection.
* QKV projection, ``getQKVmatrices`` (``attention_qkv_kernels.cu:51-122``): for row
  ``r = b*T + t`` and output feature ``j = h*d + dd``,
  ``Q[b, h, t, dd] = sum_i X[r, i] Wq[j, i] + bq[j]`` -- the weights are indexed
  ``[H*d][E]`` (``:92``) although the getter labels them ``[E, H*d]``
  (``AttentionLayer.cu:168``); likewise K and V.  The output is written in ``[B, H, T, d]``
  (``:112-120``).
* attention core: ``oracle.attention_fp64`` (``flash_attention.cu``).
* output projection, ``attentionProj`` (``attention_proj_kernels.cu:48-98``):
  ``Y[r, e] = sum_c C[r, c] Wo[e, c] + bo[e]`` with ``C[r, h*d + dd] = attn[b, h, t, dd]``
  (``:72-77``), ``Wo`` indexed ``[E][H*d]`` (``:82``).
* backward, ``AttentionLayer::backward`` (``AttentionLayer.cu:127-158``):
  - ``projBackwardWB`` (``attention_proj_kernels.cu:142-238``):
    ``dWo[e, c] += sum_r dY[r, e] C[r, c]``, ``dbo[e] += sum_r dY[r, e]``;
  - ``projBackward`` (``:240-288``): ``dC[r, c] = sum_e dY[r, e] Wo[e, c]``;
  - attention backward;
  - ``qkvBackwardWB`` (``attention_qkv_kernels.cu:171-293``):
    ``dWq[j, i] += sum_r dQ[r, j] X[r, i]``, ``dbq[j] += sum_r dQ[r, j]`` (same for K, V);
  - ``qkvBackward`` (``:295-364``): ``dX = dQ Wq + dK Wk + dV Wv``.

Departures, all deliberate: the bias gradients sum every row (the reference's kernels add
only the first row of each 32-row tile, ``attention_qkv_kernels.cu:233-237`` and
``attention_proj_kernels.cu:188,194-196``); the attention output is kept for the output
projection's backward (the reference frees it before use, ``AttentionLayer.cu:98-100``);
an optional causal mask.  Weight and bias gradients are returned as the increment the
call adds (the reference accumulates them across calls until ``zeroGrad``).
"""
from __future__ import annotations

import numpy as np

from . import attention_fp64 as attn

__all__ = ["to_rows", "from_rows", "layer_fwd", "layer_bwd", "make_layer_inputs"]


def to_rows(a: np.ndarray) -> np.ndarray:
    """[B, H, T, d] -> [B*T, H*d] (row b*T + t, column h*d + dd)."""
    b, h, t, d = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(b * t, h * d)


def from_rows(m: np.ndarray, b: int, h: int, t: int, d: int) -> np.ndarray:
    """[B*T, H*d] -> [B, H, T, d]."""
    return np.ascontiguousarray(m.reshape(b, t, h, d).transpose(0, 2, 1, 3))


def layer_fwd(x, wq, wk, wv, bq, bk, bv, wo, bo, num_heads: int, head_dim: int, causal=False):
    """x [B, T, E] -> dict(q, k, v, c, lse, y); every array float64."""
    x = np.asarray(x, dtype=np.float64)
    b, t, e = x.shape
    xr = x.reshape(b * t, e)
    proj = {}
    for name, w, bias in (("q", wq, bq), ("k", wk, bk), ("v", wv, bv)):
        m = xr @ np.asarray(w, np.float64).T + np.asarray(bias, np.float64)[None, :]
        proj[name] = from_rows(m, b, num_heads, t, head_dim)
    o, lse = attn.attention_fwd(proj["q"], proj["k"], proj["v"], causal)
    y = to_rows(o) @ np.asarray(wo, np.float64).T + np.asarray(bo, np.float64)[None, :]
    return dict(q=proj["q"], k=proj["k"], v=proj["v"], c=o, lse=lse, y=y.reshape(b, t, e))


def layer_bwd(x, wq, wk, wv, wo, fwd: dict, dy, causal=False):
    """Gradients of sum(Y * dY): dict(dx, dwq, dwk, dwv, dbq, dbk, dbv, dwo, dbo, dc, dq,
    dk, dv); every array float64."""
    x = np.asarray(x, dtype=np.float64)
    b, t, e = x.shape
    _, h, _, d = fwd["q"].shape
    xr = x.reshape(b * t, e)
    dyr = np.asarray(dy, np.float64).reshape(b * t, e)
    cr = to_rows(fwd["c"])
    out = {"dwo": dyr.T @ cr, "dbo": dyr.sum(axis=0)}
    dcr = dyr @ np.asarray(wo, np.float64)
    out["dc"] = from_rows(dcr, b, h, t, d)
    dq, dk, dv = attn.attention_bwd(fwd["q"], fwd["k"], fwd["v"], fwd["c"], out["dc"], fwd["lse"], causal)
    out.update(dq=dq, dk=dk, dv=dv)
    dx = np.zeros_like(xr)
    for name, w in (("q", wq), ("k", wk), ("v", wv)):
        gr = to_rows(out["d" + name])
        out["dw" + name] = gr.T @ xr
        out["db" + name] = gr.sum(axis=0)
        dx += gr @ np.asarray(w, np.float64)
    out["dx"] = dx.reshape(b, t, e)
    return out


def make_layer_inputs(b, t, e, h, d, seed, dtype="f32", weight_scale=None, bias_std=0.1):
    """Seeded x [B, T, E] ~ N(0, 1), weights ~ N(0, 1/E) (Wq/Wk/Wv [H*d, E]) and
    N(0, 1/(H*d)) (Wo [E, H*d]) -- the scaling the reference's test uses
    (``test_flash_attention.py:20-23``) -- biases ~ N(0, bias_std^2), dY ~ N(0, 1); all
    cast to the run's dtype and returned as float32 arrays (float64 for dtype "f64")."""
    rng = np.random.default_rng(seed)
    hd = h * d
    ws_in = weight_scale if weight_scale is not None else 1.0 / np.sqrt(e)
    ws_out = weight_scale if weight_scale is not None else 1.0 / np.sqrt(hd)
    arrs = dict(
        x=rng.standard_normal((b, t, e)),
        wq=rng.standard_normal((hd, e)) * ws_in,
        wk=rng.standard_normal((hd, e)) * ws_in,
        wv=rng.standard_normal((hd, e)) * ws_in,
        bq=rng.standard_normal(hd) * bias_std,
        bk=rng.standard_normal(hd) * bias_std,
        bv=rng.standard_normal(hd) * bias_std,
        wo=rng.standard_normal((e, hd)) * ws_out,
        bo=rng.standard_normal(e) * bias_std,
        dy=rng.standard_normal((b, t, e)),
    )
    cast = {"bf16": attn.round_to_bf16, "f16": attn.round_to_f16, "f64": lambda a: a,
            "f32": lambda a: a.astype(np.float32)}[dtype]
    return {k: cast(v) for k, v in arrs.items()}
