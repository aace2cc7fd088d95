"""ctattn_bwd_noalloc: the backward with its workspace in the library's static scratch.

The entry point allocates nothing; its results must equal ctattn_bwd's (same kernels, the
workspace only moves), on two calls in a row with the second problem smaller than the first
(the scratch keeps the first call's contents), under the AUTO and DETERMINISTIC policies, on
the MFMA kernels (fp32, bf16, fp64; d = 48 runs padded onto the d = 64 fp32 kernels) and the
generic kernels (d = 160), on torch's current stream and on a second stream; a bf16 d = 128
problem whose dS tiles exceed the scratch takes the recomputing dQ kernel; and a warmed-up
call changes the device's free memory by nothing.  Bar: fp32 / fp64 max-abs <= 1e-4 (fp32 dQ is summed with atomics under AUTO,
so it may differ in the last bits), bf16 max-rel <= 2e-2, and dK / dV -- written without
atomics on every path -- bitwise equal.
"""
import sys

import numpy as np
import pytest
import torch

import cudatransformer_amd as ct
from cudatransformer_amd import _capi

DEV = "cuda:0"
SHAPES = [(2, 4, 300, None), (1, 2, 100, None)]  # second call smaller than the first
CASES = [(torch.float32, 64), (torch.bfloat16, 128), (torch.float64, 64), (torch.float32, 48),
         (torch.float32, 160)]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_noalloc_rejects_problems_beyond_the_scratch():
    """Host-side check, before any GPU work (runs without a GPU): 16 Mi rows of bf16 need
    128 MiB of scratch, more than the 32 MiB buffer."""
    lib = _capi.load()
    rc = lib.ctattn_bwd_noalloc(_capi.BF16, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 32, 1 << 19, 128, 1, None)
    assert rc == 1 and "scratch" in _capi.last_error()
    assert lib.ctattn_bwd_workspace_bytes(_capi.BF16, 1, 32, 1 << 19, 128, 1) > _capi.NOALLOC_SCRATCH_BYTES


@pytest.mark.gpu
@pytest.mark.parametrize("policy", [_capi.POLICY_AUTO, _capi.POLICY_DETERMINISTIC], ids=["auto", "deterministic"])
@pytest.mark.parametrize("dtype,d", CASES, ids=lambda x: str(x).replace("torch.", ""))
def test_noalloc_matches_bwd(dtype, d, policy):
    prev = _capi.set_policy(policy)
    try:
        side = torch.cuda.Stream()  # default priority
        for i, (b, h, t, _) in enumerate(SHAPES):
            shape = (b, h, t, d)
            say(f"noalloc {dtype} shape={shape} policy={policy} call={i}")
            g = torch.Generator(device=DEV).manual_seed(90 + i)
            std = 0.5 if dtype == torch.bfloat16 else 1.0
            q, k, v, do = ((std * torch.randn(shape, generator=g, device=DEV, dtype=torch.float64)).to(dtype)
                           for _ in range(4))
            causal = i == 0
            o, lse = ct.flash_attn_fwd(q, k, v, causal)
            ref = ct.flash_attn_bwd(q, k, v, o, do, lse, causal)
            stream = side if i == 1 else None
            if stream is not None:
                stream.wait_stream(torch.cuda.current_stream())
            got = _capi.flash_attn_bwd_noalloc(q, k, v, o, do, lse, causal, stream=stream)
            torch.cuda.synchronize()
            for name, a, r in zip(("dq", "dk", "dv"), got, ref):
                x, y = a.double().cpu().numpy(), r.double().cpu().numpy()
                assert np.all(np.isfinite(x)), name
                err = float(np.max(np.abs(x - y)))
                if dtype == torch.bfloat16:
                    assert err / max(float(np.max(np.abs(y))), 1e-30) <= 2e-2, (name, err)
                else:
                    assert err <= 1e-4, (name, err)
                if name != "dq" or dtype != torch.float32 or policy == _capi.POLICY_DETERMINISTIC:
                    assert np.array_equal(x, y), f"{name}: not bitwise equal to ctattn_bwd ({err:.3e})"
    finally:
        _capi.set_policy(prev)


@pytest.mark.gpu
def test_noalloc_recompute_fallback_and_no_allocation():
    """B1 H8 T4096 d128 bf16 causal: 135 MB of dS tiles, more than the 32 MiB scratch, so the
    entry point runs the recomputing dQ kernel -- the path ctattn_bwd takes with its default
    workspace at this shape -- and matches it bitwise.  A second call with preallocated
    outputs leaves hipMemGetInfo's free memory unchanged."""
    shape, causal = (1, 8, 4096, 128), True
    say(f"noalloc bf16 recompute fallback shape={shape}")
    nt = 4096 // 32
    assert 8 * nt * (nt + 1) // 2 * 2048 > _capi.NOALLOC_SCRATCH_BYTES
    g = torch.Generator(device=DEV).manual_seed(97)
    q, k, v, do = ((0.5 * torch.randn(shape, generator=g, device=DEV)).to(torch.bfloat16) for _ in range(4))
    o, lse = ct.flash_attn_fwd(q, k, v, causal)
    ref = ct.flash_attn_bwd(q, k, v, o, do, lse, causal)
    outs = tuple(torch.empty_like(q) for _ in range(3))
    _capi.flash_attn_bwd_noalloc(q, k, v, o, do, lse, causal, *outs)
    torch.cuda.synchronize()
    for name, a, r in zip(("dq", "dk", "dv"), outs, ref):
        assert torch.equal(a, r), f"{name}: not bitwise equal to ctattn_bwd's default path"
    free0 = torch.cuda.mem_get_info()[0]
    _capi.flash_attn_bwd_noalloc(q, k, v, o, do, lse, causal, *outs)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
