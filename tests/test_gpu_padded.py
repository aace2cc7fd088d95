"""Head dims without an MFMA kernel of their own (d <= 128, not 32 / 64 / 128): ctattn_fwd and
ctattn_bwd run the MFMA kernels of the next width (32, 64 or 128) on zero-padded copies, with
the scores scaled by 1/sqrt(d) of the real head dim, and copy O, dQ, dK, dV back.

Checked through the C-ABI against the fp64 oracle on the same storage-rounded inputs, at the
tolerances of the native head dims (fp32 max-abs 1e-4; bf16 2e-2, fp16 4e-3, fp64 1e-10
relative to the largest value), against the generic kernels (POLICY_GENERIC, which take any
d), bitwise across two runs under POLICY_DETERMINISTIC, and with a caller stream.
"""
import sys

import numpy as np
import pytest
import torch

import cudatransformer_amd as ct
from oracle import attention_fp64 as ora

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16, "f64": torch.float64}
REL = {"bf16": 2e-2, "f16": 4e-3, "f64": 1e-10}
F32_ABS = 1e-4


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run(q, k, v, do, causal, name, stream=None):
    td = TORCH[name]
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a, np.float64)).to(DEV).to(td) for a in (q, k, v, do))
    o, lse = ct.flash_attn_fwd(tq, tk, tv, causal)
    dq, dk, dv = ct.flash_attn_bwd(tq, tk, tv, o, tdo, lse, causal)
    torch.cuda.synchronize()
    f = lambda t: t.double().cpu().numpy()  # noqa: E731
    return {"o": f(o), "lse": f(lse), "dq": f(dq), "dk": f(dk), "dv": f(dv)}


def check(got, want, name, ctx):
    # dQ / dK of a row that sees one key vanish in exact arithmetic; their scale then falls
    # back to 1e-4 of the dV scale (as in the native-head-dim parity tests).
    dv_scale = float(np.max(np.abs(want["dv"])))
    for key in ("o", "lse", "dq", "dk", "dv"):
        g, w = got[key], want[key]
        assert g.shape == w.shape, (ctx, key)
        assert np.all(np.isfinite(g)), f"{ctx} {key}: non-finite"
        err = float(np.max(np.abs(g - w)))
        if name == "f32":
            assert err <= F32_ABS, f"{ctx} {key}: max abs err {err:.3e}"
        else:
            floor = 1e-4 * dv_scale if key in ("dq", "dk") else 0.0
            scale = max(float(np.max(np.abs(w))), floor, 1e-30)
            assert err <= REL[name] * scale, f"{ctx} {key}: err {err:.3e} vs scale {scale:.3e}"


@pytest.mark.parametrize("d", [8, 16, 48, 80, 96, 100, 120])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("name", ["f32", "bf16", "f16", "f64"])
def test_padded_head_dims_match_oracle(name, causal, d):
    shape = (2, 3, 150, d)  # ragged T: partial key and query blocks
    say(f"padded head dim {name} causal={causal} shape={shape}")
    std = 0.5 if name == "bf16" else 1.0
    q, k, v, do = ora.make_inputs(shape, seed=500 + d, std=std, dtype=name)
    want = ora.attention_fwd_bwd(*ora.cast_inputs((q, k, v, do), name), causal)
    check(run(q, k, v, do, causal, name), want, name, f"{name} d={d} causal={causal}")


@pytest.mark.parametrize("d", [48, 96])
@pytest.mark.parametrize("name", ["f32", "bf16"])
def test_padded_matches_generic_kernels(name, d):
    """The padded MFMA path and the generic kernels (which take d as it is) agree."""
    shape = (1, 4, 257, d)
    say(f"padded vs generic {name} shape={shape}")
    q, k, v, do = ora.make_inputs(shape, seed=600 + d, std=0.5, dtype=name)
    padded = run(q, k, v, do, True, name)
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        generic = run(q, k, v, do, True, name)
    finally:
        ct.set_policy(prev)
    for key in padded:
        scale = max(float(np.max(np.abs(generic[key]))), 1e-30)
        tol = 1e-5 if name == "f32" else 2e-2
        err = float(np.max(np.abs(padded[key] - generic[key])))
        assert err <= tol * scale, f"{name} d={d} {key}: {err:.3e} vs scale {scale:.3e}"


@pytest.mark.parametrize("name", ["f32", "bf16"])
def test_padded_deterministic_policy_is_bitwise_reproducible(name):
    shape = (1, 2, 1100, 80)  # fp32: past 8 key blocks of 128, the query-major dQ kernel
    say(f"padded deterministic {name} shape={shape}")
    q, k, v, do = ora.make_inputs(shape, seed=700, std=0.5, dtype=name)
    prev = ct.set_policy(ct.POLICY_DETERMINISTIC)
    try:
        r1 = run(q, k, v, do, True, name)
        r2 = run(q, k, v, do, True, name)
    finally:
        ct.set_policy(prev)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key


def test_padded_on_a_side_stream():
    """The padded copies and their stream-ordered scratch follow the caller's stream."""
    shape = (2, 2, 200, 72)
    q, k, v, do = ora.make_inputs(shape, seed=710)
    want = ora.attention_fwd_bwd(q, k, v, do, True)
    side = torch.cuda.Stream()  # default priority
    tq, tk, tv, tdo = (torch.from_numpy(a).to(DEV) for a in (q, k, v, do))
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        o, lse = ct.flash_attn_fwd(tq, tk, tv, True)
        dq, dk, dv = ct.flash_attn_bwd(tq, tk, tv, o, tdo, lse, True)
    side.synchronize()
    got = {n: t.double().cpu().numpy() for n, t in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))}
    check(got, want, "f32", "side stream d=72")
