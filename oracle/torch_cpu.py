"""PyTorch-CPU scaled-dot-product attention: library cross-check and CPU baseline.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

``torch.nn.functional.scaled_dot_product_attention`` is the routine the reference's own
test compares against (``test_flash_attention.py:49``, there with ``is_causal=False``).
In fp64 with autograd it is an independent library check of ``attention_fp64``; in fp32
on all host cores it is the multi-threaded CPU figure that ``bench.py`` reports beside its
CPU baseline (the C restatement ``attn_online.c``).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def fwd_bwd(q, k, v, do, causal: bool, dtype=torch.float64):
    """Returns dict(o, lse, dq, dk, dv) as numpy arrays in ``dtype``.

    LSE is not exposed by SDPA; it is recomputed densely in the same dtype.
    """
    qt, kt, vt = (torch.tensor(np.asarray(a), dtype=dtype, requires_grad=True) for a in (q, k, v))
    dot = torch.tensor(np.asarray(do), dtype=dtype)
    o = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)
    o.backward(dot)
    with torch.no_grad():
        s = qt @ kt.transpose(-1, -2) / np.sqrt(qt.shape[-1])
        if causal:
            t = s.shape[-1]
            s = s.masked_fill(torch.ones(t, t, dtype=torch.bool).triu(1), float("-inf"))
        lse = torch.logsumexp(s, dim=-1)
    return {
        "o": o.detach().numpy(),
        "lse": lse.numpy(),
        "dq": qt.grad.numpy(),
        "dk": kt.grad.numpy(),
        "dv": vt.grad.numpy(),
    }


def time_fwd_bwd(shape, causal: bool, seconds: float = 10.0, threads: int | None = None,
                 dtype=torch.float32, seed: int = 2, max_reps: int = 200):
    """Times SDPA fwd+bwd on CPU tensors for about ``seconds`` of work.

    One warm-up, then repetitions until ``seconds`` elapsed (at least 3).  Returns
    ``(median_seconds, reps, threads_used)``.
    """
    import os
    import time

    if threads is None:
        threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(shape, generator=g, dtype=dtype) for _ in range(4))

    def step():
        qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
        o = F.scaled_dot_product_attention(qq, kk, vv, is_causal=causal)
        o.backward(do)

    step()
    times = []
    t_end = time.perf_counter() + seconds
    while (len(times) < 3 or time.perf_counter() < t_end) and len(times) < max_reps:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times), threads
