"""Writes the golden attention fixtures in this directory.

The reference holds no golden vectors for this path (its only check is
test_flash_attention.py:52, unseeded).  These fixtures are generated from the fp64 oracle
(oracle/attention_fp64.py) and, before being written, cross-checked against torch's
scaled_dot_product_attention in fp64 with autograd (the comparator of the reference's
own test).  Expected outputs are stored as float32 (rounding <= 6e-8 relative, far
inside the 1e-4 / 2e-2 tolerances).  Inputs follow the synthetic-input recipe: numpy default_rng(seed), drawn in
fp64 in the order Q, K, V, dO, scaled, then rounded to the storage dtype.

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention_fp64 as ora  # noqa: E402
from oracle import torch_cpu  # noqa: E402

# name: (shape [B,H,T,d], seed, std, dtype)
CASES = {
    "c1_b1h4t128d32_f32": ((1, 4, 128, 32), 1, 1.0, "f32"),
    "ragged_b1h2t40d16_f32": ((1, 2, 40, 16), 21, 1.0, "f32"),
    "single_b2h1t1d32_f32": ((2, 1, 1, 32), 22, 1.0, "f32"),
    "ragged_b1h1t100d64_f32": ((1, 1, 100, 64), 23, 1.0, "f32"),
    "small_b1h2t64d64_bf16": ((1, 2, 64, 64), 4, 0.5, "bf16"),
}


def make(name, shape, seed, std, dtype):
    q, k, v, do = ora.make_inputs(shape, seed, std=std, dtype=dtype)
    out = {"q": q, "k": k, "v": v, "do": do}
    for causal in (False, True):
        r = ora.attention_fwd_bwd(q, k, v, do, causal)
        t = torch_cpu.fwd_bwd(q, k, v, do, causal)
        for key in ("o", "lse", "dq", "dk", "dv"):
            err = float(np.max(np.abs(r[key] - t[key])))
            assert err < 1e-10, f"{name} causal={causal} {key}: oracle vs torch {err}"
            out[f"{key}_{'causal' if causal else 'full'}"] = r[key].astype(np.float32)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    for name, args in CASES.items():
        make(name, *args)
