"""Sizes past the 32-bit limits the reference is bound by, on the GPU through the C-ABI.

The reference indexes its tensors with ``int`` offsets (``flash_attention.cu:77-78``:
``batchIdx * numHeads * seqLen * headDim + ...``), which wrap once a tensor holds 2^31
elements.  This build computes element offsets in int64 and launches its row-parallel
kernels with grid-stride loops, so both limits are gone:

* more than 2^31 elements per tensor on the MFMA kernels (fp32 and bf16): the first and the
  last (b, h) slice -- whose element offsets are above 2^31 -- against the fp64 oracle; bf16
  d = 128 both with the recomputing dQ kernel and with the dS tiles stored in the workspace
  (2.7 GB of tiles at 131073 heads of T = 128);
* more than 2^26 rows on the generic kernels (one wave per row: 2^26 rows x 64 lanes is the
  2^32 work-item limit of one launch), again first and last slices against the oracle.

Inputs are generated on the GPU (seeded); only the checked slices come back to the host.
"""
import sys

import numpy as np
import pytest
import torch

import cudatransformer_amd as ct
from oracle import attention_fp64 as ora

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check_slices(tensors, causal, bh_list, dtype, ctx):
    """tensors: dict of the GPU inputs and results ([B, H, T, d]; lse [B, H, T]).  Compares
    the (b, h) slices in bh_list against the oracle run on the same (rounded) inputs."""
    for b, h in bh_list:
        f = lambda name: tensors[name][b:b + 1, h:h + 1].float().cpu().numpy().astype(np.float64)  # noqa: E731
        q, k, v, do = (f(n) for n in ("q", "k", "v", "do"))
        want = ora.attention_fwd_bwd(q, k, v, do, causal)
        for name in ("o", "lse", "dq", "dk", "dv"):
            g, w = f(name), want[name]
            err = float(np.max(np.abs(g - w)))
            if dtype == torch.float32:
                assert err <= 1e-4, f"{ctx} slice ({b}, {h}) {name}: max abs err {err:.3e}"
            else:
                rel = err / max(float(np.max(np.abs(w))), 1e-30)
                assert rel <= 2e-2, f"{ctx} slice ({b}, {h}) {name}: rel err {rel:.3e}"


def run_big(shape, causal, dtype, std, seed, fastest=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = {n: (std * torch.randn(shape, generator=g, device=DEV, dtype=torch.float32)).to(dtype)
         for n in ("q", "k", "v", "do")}
    o, lse = ct.flash_attn_fwd(t["q"], t["k"], t["v"], causal)
    ws = None
    if fastest:
        ws = torch.empty(ct._capi.bwd_workspace_bytes(dtype, *shape, causal, fastest=True), dtype=torch.uint8,
                         device=DEV)
    dq, dk, dv = ct.flash_attn_bwd(t["q"], t["k"], t["v"], o, t["do"], lse, causal, workspace=ws)
    torch.cuda.synchronize()
    t.update(o=o, lse=lse, dq=dq, dk=dk, dv=dv)
    return t


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_more_than_2_31_elements_mfma(dtype):
    """B2050 H8 T1024 d128 causal: 2,149,580,800 elements per tensor (> 2^31); the last
    slice starts at element 2,149,449,728."""
    shape = (2050, 8, 1024, 128)
    n = shape[0] * shape[1] * shape[2] * shape[3]
    assert n > 2 ** 31 and (shape[0] * shape[1] - 1) * shape[2] * shape[3] > 2 ** 31
    say(f"large MFMA problem {shape} {dtype}")
    t = run_big(shape, True, dtype, 1.0 if dtype == torch.float32 else 0.5, seed=71)
    check_slices(t, True, [(0, 0), (shape[0] - 1, shape[1] - 1), (shape[0] // 2, 3)], dtype,
                 f"{shape} {dtype}")
    del t
    torch.cuda.empty_cache()


def test_more_than_2_31_elements_bf16_ds_tiles():
    """B1 H131073 T128 d128 bf16 causal: 2,147,500,032 elements per tensor (> 2^31) with the
    dS tiles in the workspace (131073 heads x 10 tiles x 2 KiB = 2.7 GB, under the 4 GiB limit),
    so the dK/dV kernel's tile stores and the dQ kernel's tile reads use 64-bit offsets; the
    first, middle and last heads against the oracle."""
    shape = (1, 131073, 128, 128)
    n = shape[1] * shape[2] * shape[3]
    assert n > 2 ** 31
    nt = shape[2] // 32
    ds_bytes = shape[1] * nt * (nt + 1) // 2 * 2048
    assert 2 ** 31 < ds_bytes <= 4 << 30
    rows = shape[1] * shape[2]
    full = ct._capi.bwd_workspace_bytes(torch.bfloat16, *shape, True, fastest=True)
    assert full == 2 * ((rows * 4 + 255) // 256 * 256) + ds_bytes  # delta, -LSE log2(e), the tiles
    say(f"large bf16 problem with dS tiles {shape}")
    t = run_big(shape, True, torch.bfloat16, 0.5, seed=73, fastest=True)
    check_slices(t, True, [(0, 0), (0, shape[1] // 2), (0, shape[1] - 1)], torch.bfloat16, f"{shape} dS tiles")
    del t
    torch.cuda.empty_cache()


def test_more_than_2_26_rows_generic():
    """The generic kernels (POLICY_GENERIC; d = 8 would otherwise run padded on the MFMA
    kernels) at B (2^22 + 3) H1 T16 = 2^26 + 48 rows, past the 2^32 work-items one
    row-per-wave launch could hold."""
    shape = ((1 << 22) + 3, 1, 16, 8)
    rows = shape[0] * shape[1] * shape[2]
    assert rows * 64 > 2 ** 32
    say(f"large generic problem {shape}")
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        for causal in (True, False):
            t = run_big(shape, causal, torch.float32, 1.0, seed=72)
            check_slices(t, causal, [(0, 0), (shape[0] - 1, 0), (shape[0] // 3, 0)], torch.float32,
                         f"{shape} causal={causal}")
            del t
    finally:
        ct.set_policy(prev)
    torch.cuda.empty_cache()
