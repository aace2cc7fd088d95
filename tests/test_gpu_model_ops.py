"""The layers around attention in libctattn.so, op by op through the C-ABI (ctypes), against
float64 references computed by torch on the CPU.

Each op follows a reference kernel (linear_kernels.cu, layer_norm_kernels.cu, relu / gelu /
sigmoid / tanh_kernels.cu, embedding_kernels.cu, loss_kernels.cu, adam_kernels.cu); the
float64 formulas here are the textbook definitions those kernels implement (GELU in its tanh
form, LayerNorm with the biased variance and eps inside the square root, softmax with a
temperature, cross-entropy -log p[target] / N).  Tolerances are stated per test: fp32
storage is held to a few fp32 ulps of the result's scale, bf16 and fp16 storage to their
rounding of the inputs and output, fp64 storage (fp64 arithmetic) to 1e-12 of the result's
scale.  Integer work (embedding lookup) is bit-exact.
"""
import math

import numpy as np

import pytest
import torch
import torch.nn.functional as F

from cudatransformer_amd import _capi

pytestmark = pytest.mark.gpu
DEV = "cuda"
F64 = torch.float64


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(shape, seed, scale=1.0):
    return torch.randn(shape, generator=_gen(seed), dtype=F64) * scale


def _dev(t, dtype):
    return t.to(dtype).contiguous().to(DEV)


def _as64(t_dev_or_cpu, dtype):
    """The values the GPU actually received (rounded to the storage dtype), as float64."""
    return t_dev_or_cpu.to(dtype).to(F64).cpu()


def _close(got, ref, rel, what, abs_floor=0.0):
    got = got.detach().to(F64).cpu()
    scale = float(ref.abs().max()) if ref.numel() else 0.0
    err = float((got - ref).abs().max()) if ref.numel() else 0.0
    assert err <= rel * scale + abs_floor, f"{what}: max err {err:.3e} vs scale {scale:.3e} (rel {rel})"


TOL = {torch.float32: 2e-5, torch.bfloat16: 1.6e-2, torch.float16: 2e-3, F64: 1e-12}
DTYPES = [torch.float32, torch.bfloat16, torch.float16, F64]
DT_IDS = ["f32", "bf16", "f16", "f64"]


def _stat_tol(dtype):
    """Tolerance of a statistic (row mean, rstd, loss): fp64 for fp64 storage, else fp32."""
    return TOL[F64] if dtype == F64 else TOL[torch.float32]


# ---- linear --------------------------------------------------------------------------------

# (100, 96, 256): rows that no tile divides; (384, 128, 256): every product on the fast load
# path; (2048, 64, 96): a weight gradient split over many K ranges.
LINEAR_SHAPES = [(1, 1, 1), (37, 130, 65), (256, 384, 384), (300, 65, 1536), (64, 4, 8), (100, 96, 256),
                 (384, 128, 256), (2048, 64, 96)]


@pytest.fixture(params=[_capi.POLICY_AUTO, _capi.POLICY_GENERIC], ids=["lin_gemm", "proj_gemm"])
def gemm_path(request):
    """AUTO sends the fp32 linear products to the split-K-in-workgroup GEMMs (linear_gemm.hip)
    where their shape allows it, GENERIC keeps every product on the projection GEMM family
    (proj_gemm.hip): both paths are checked."""
    prev = _capi.set_policy(request.param)
    yield request.param
    _capi.set_policy(prev)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("mnk", LINEAR_SHAPES)
@pytest.mark.parametrize("bias", [True, False])
def test_linear_fwd_bwd(dtype, mnk, bias, gemm_path):
    m, n, k = mnk
    print(f"linear {dtype} M={m} N={n} K={k} bias={bias} policy={gemm_path}", flush=True)
    x = _dev(_randn((m, k), 1), dtype)
    w = _dev(_randn((n, k), 2, 1 / math.sqrt(k)), dtype)
    b = _dev(_randn((n,), 3), dtype) if bias else None
    dy = _dev(_randn((m, n), 4), dtype)
    dw0 = _randn((n, k), 5)
    db0 = _randn((n,), 6)
    dw = _dev(dw0, dtype)
    db = _dev(db0, dtype) if bias else None

    y = _capi.linear_fwd(x, w, b)
    dx = _capi.linear_bwd(x, w, dy, dw, db)
    torch.cuda.synchronize()

    x64, w64, dy64 = _as64(x, dtype), _as64(w, dtype), _as64(dy, dtype)
    ref_y = x64 @ w64.T + (_as64(b, dtype) if bias else 0.0)
    _close(y, ref_y, TOL[dtype], "y")
    _close(dx, dy64 @ w64, TOL[dtype], "dx")
    # dw / db accumulate into what the buffers held.
    _close(dw, _as64(dw0, dtype) + dy64.T @ x64, TOL[dtype], "dw")
    if bias:
        _close(db, _as64(db0, dtype) + dy64.sum(0), TOL[dtype], "db")


# Shapes on linear_gemm.hip covering its launch plans (fp32 / 16-bit; forward, dX, dW):
#   (4096, 1536, 384)  fp32 forward on the shared-tile kernel (768 128 x 64 tiles, GELU-MLP
#                      width); dW split 4 ways; 16-bit forward shared-tile, two-chunk stages
#   (4096, 384, 1536)  forward / dW four waves per tile; dX 3072 tiles, one wave
#   (8192, 1024, 1024) fp32 forward shared-tile, dX one wave per tile, 3 stages, dW 64 x 64 tiles
#                      of 8 waves; 16-bit: every product shared-tile (dW unsplit from 256 tiles)
#   (1008, 208, 1008)  ragged tiles in M, N and K-chunk count on all three products
#   (64, 16, 4096)     dX with one K chunk for four waves (three waves add a zero tile)
#   (8192, 64, 64)     dW split 8 ways on 8-wave 64 x 32 tiles (8 of the 512 K chunks per wave)
#   (4096, 1152, 384)  the QKV-width product of the NanoGPT configuration (576 tiles: lin_kernel)
#   (8100, 1024, 992)  ragged M (forward) and N (dX); 16-bit forward with one-chunk stages
#   (2000, 1984, 2016) 16-bit shared-tile forward and dX with ragged M and N, one- and
#                      two-chunk stages
#   (2048, 2048, 2048) 16-bit dW on the shared-tile kernel without a K split (256 tiles)
#   (4096, 2050, 512)  N not a multiple of 4: the shared-tile kernel's element-wise epilogue
LIN_SHAPES = [(4096, 1536, 384), (4096, 384, 1536), (8192, 1024, 1024), (1008, 208, 1008), (64, 16, 4096),
              (8192, 64, 64), (4096, 1152, 384), (8100, 1024, 992), (2000, 1984, 2016), (2048, 2048, 2048),
              (4096, 2050, 512)]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("mnk", LIN_SHAPES)
def test_linear_plans(mnk, dt):
    """Every launch configuration of the linear GEMMs (fp32 MFMA for fp32, the 16-bit MFMA for
    bf16 / fp16 storage) against fp64 on the same rounded inputs, bias on, dW / db accumulating
    into non-zero buffers."""
    m, n, k = mnk
    print(f"linear plans M={m} N={n} K={k} {dt}", flush=True)
    x = _dev(_randn((m, k), 21), dt)
    w = _dev(_randn((n, k), 22, 1 / math.sqrt(k)), dt)
    b = _dev(_randn((n,), 23), dt)
    dy = _dev(_randn((m, n), 24), dt)
    dw0, db0 = _randn((n, k), 25), _randn((n,), 26)
    dw, db = _dev(dw0, dt), _dev(db0, dt)
    y = _capi.linear_fwd(x, w, b)
    dx = _capi.linear_bwd(x, w, dy, dw, db)
    torch.cuda.synchronize()
    x64, w64, dy64 = _as64(x, dt), _as64(w, dt), _as64(dy, dt)
    _close(y, x64 @ w64.T + _as64(b, dt), TOL[dt], "y")
    _close(dx, dy64 @ w64, TOL[dt], "dx")
    _close(dw, _as64(dw0, dt) + dy64.T @ x64, TOL[dt], "dw")
    _close(db, _as64(db0, dt) + dy64.sum(0), TOL[dt], "db")


# (B, T, E, H, d): products of at least 256 128 x 128 tiles take the 16-bit shared-tile GEMM
# (fp32: forward products of at least 768 128 x 64 tiles, the B8 shape's head-split output
# projection among them); d = 64 stages two K chunks per head, d = 32 one; T = 700 puts batch
# boundaries inside tiles; d = 12 writes a head-split output in 4-column groups.
# The last three put odd and small T and small d under the head-split row / column offsets
# (divisions by T and d done as multiply-high and shift on the device).
PROJ_SHAPES = [(4, 1024, 1024, 16, 64), (2, 2048, 1024, 32, 32), (3, 700, 768, 12, 64), (8, 1024, 1024, 16, 64),
               (4, 1024, 512, 32, 12), (2, 1025, 256, 8, 32), (3, 17, 128, 4, 32), (2, 333, 64, 16, 4)]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("dims", PROJ_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_projection_products_16bit_large(dims, dt):
    """The attention layer's projections at sizes of the shared-tile GEMM (head-split Q / K / V /
    C operands and outputs, dX summing three K segments) against float64 products of the same
    rounded inputs."""
    b, t, e, h, d = dims
    hd = h * d
    print(f"projection products {dims} {dt}", flush=True)
    x = _dev(_randn((b, t, e), 30), dt)
    ws = [_dev(_randn((hd, e), 31 + i, 1 / math.sqrt(e)), dt) for i in range(3)]
    bs = [_dev(_randn((hd,), 34 + i), dt) for i in range(3)]
    qkv = _capi.qkv_proj_fwd(x, *ws, *bs, h, d)
    x64 = _as64(x, dt).reshape(b * t, e)

    def heads(r):  # [B*T, H*d] rows -> [B, H, T, d]
        return r.reshape(b, t, h, d).permute(0, 2, 1, 3)

    def rows(g):  # [B, H, T, d] -> [B*T, H*d] rows, float64
        return _as64(g, dt).permute(0, 2, 1, 3).reshape(b * t, hd)

    for o, w, bb, n in zip(qkv, ws, bs, "qkv"):
        _close(o, heads(x64 @ _as64(w, dt).T + _as64(bb, dt)), TOL[dt], n)
    c = _dev(_randn((b, h, t, d), 40), dt)
    wo = _dev(_randn((e, hd), 41, 1 / math.sqrt(hd)), dt)
    bo = _dev(_randn((e,), 42), dt)
    y = _capi.out_proj_fwd(c, wo, bo)
    _close(y, (rows(c) @ _as64(wo, dt).T + _as64(bo, dt)).reshape(b, t, e), TOL[dt], "y")
    dy = _dev(_randn((b, t, e), 43), dt)
    dwo, dbo = torch.zeros_like(wo), torch.zeros_like(bo)
    dc = _capi.out_proj_bwd(c, dy, wo, dwo, dbo)
    dy64 = _as64(dy, dt).reshape(b * t, e)
    _close(dc, heads(dy64 @ _as64(wo, dt)), TOL[dt], "dc")
    _close(dwo, dy64.T @ rows(c), TOL[dt], "dwo")
    _close(dbo, dy64.sum(0), TOL[dt], "dbo")
    grads = [_dev(_randn((b, h, t, d), 50 + i), dt) for i in range(3)]
    dw = tuple(torch.zeros_like(w) for w in ws)
    db = tuple(torch.zeros_like(bb) for bb in bs)
    dx = _capi.qkv_proj_bwd(x, *grads, *ws, dw=dw, db=db)
    torch.cuda.synchronize()
    _close(dx, sum(rows(g) @ _as64(w, dt) for g, w in zip(grads, ws)).reshape(b, t, e), TOL[dt], "dx")
    for g, dwi, dbi, n in zip(grads, dw, db, "qkv"):
        _close(dwi, rows(g).T @ x64, TOL[dt], "dw" + n)
        _close(dbi, rows(g).sum(0), TOL[dt], "db" + n)


def test_linear_fp32_bitwise_repeatable():
    """The fp32 linear products use no atomics: a split-K weight gradient and the forward /
    dX are bitwise equal across calls."""
    m, n, k = 4096, 384, 384
    x = _dev(_randn((m, k), 27), torch.float32)
    w = _dev(_randn((n, k), 28), torch.float32)
    dy = _dev(_randn((m, n), 29), torch.float32)
    outs = []
    for _ in range(3):
        dw = torch.zeros(n, k, device="cuda")
        y = _capi.linear_fwd(x, w)
        dx = _capi.linear_bwd(x, w, dy, dw, None)
        torch.cuda.synchronize()
        outs.append((y.cpu(), dx.cpu(), dw.cpu()))
    for o in outs[1:]:
        for a, b_ in zip(outs[0], o):
            assert torch.equal(a, b_)


def test_linear_bwd_skips_and_empty():
    x = _dev(_randn((16, 8), 7), torch.float32)
    w = _dev(_randn((12, 8), 8), torch.float32)
    dy = _dev(_randn((16, 12), 9), torch.float32)
    assert _capi.linear_bwd(x, w, dy, None, None, want_dx=False) is None
    dx = _capi.linear_bwd(x, w, dy)
    torch.cuda.synchronize()
    _close(dx, _as64(dy, torch.float32) @ _as64(w, torch.float32), TOL[torch.float32], "dx only")
    y = _capi.linear_fwd(x[:0], w)
    assert y.shape == (0, 12)


# ---- layernorm -----------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("nd", [(1, 32), (7, 65), (300, 384), (33, 1536)])
def test_layernorm_fwd_bwd(dtype, nd):
    n, d = nd
    print(f"layernorm {dtype} N={n} D={d}", flush=True)
    x = _dev(_randn((n, d), 10, 3.0) + 1.5, dtype)
    g = _dev(1.0 + 0.1 * _randn((d,), 11), dtype)
    b = _dev(0.1 * _randn((d,), 12), dtype)
    dy = _dev(_randn((n, d), 13), dtype)
    dg0, db0 = _randn((d,), 14), _randn((d,), 15)
    dg, db = _dev(dg0, dtype), _dev(db0, dtype)

    y, mean, rstd = _capi.layernorm_fwd(x, g, b, 1e-5)
    dx = _capi.layernorm_bwd(x, g, dy, mean, rstd, dg, db)
    torch.cuda.synchronize()

    x64 = _as64(x, dtype).requires_grad_(True)
    g64 = _as64(g, dtype).requires_grad_(True)
    b64 = _as64(b, dtype).requires_grad_(True)
    ref = F.layer_norm(x64, (d,), g64, b64, 1e-5)
    ref.backward(_as64(dy, dtype))
    _close(y, ref.detach(), TOL[dtype], "y")
    assert mean.dtype == rstd.dtype == _capi._stat_dtype(dtype)
    _close(mean, x64.detach().mean(-1), _stat_tol(dtype), "mean")
    _close(rstd, 1 / torch.sqrt(x64.detach().var(-1, unbiased=False) + 1e-5), _stat_tol(dtype), "rstd")
    _close(dx, x64.grad, TOL[dtype] * 2, "dx")
    _close(dg, _as64(dg0, dtype) + g64.grad, TOL[dtype] * 2, "dgamma")
    _close(db, _as64(db0, dtype) + b64.grad, TOL[dtype] * 2, "dbeta")


def test_layernorm_bwd_is_deterministic():
    x = _dev(_randn((4099, 384), 16), torch.float32)
    g = _dev(_randn((384,), 17), torch.float32)
    dy = _dev(_randn((4099, 384), 18), torch.float32)
    _, mean, rstd = _capi.layernorm_fwd(x, g, torch.zeros_like(g))
    outs = []
    for _ in range(2):
        dg, db = torch.zeros_like(g), torch.zeros_like(g)
        _capi.layernorm_bwd(x, g, dy, mean, rstd, dg, db)
        outs.append((dg.cpu(), db.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("nd", [(4096, 384), (77, 96), (300, 1000), (65, 1024), (40, 1100)])
def test_layernorm_bwd_one_pass_equals_two(dtype, nd):
    """dx with dgamma / dbeta in one pass (D <= 1024: one workgroup per 32-row chunk, the
    partial sums kept per lane) against dx alone and dgamma / dbeta alone (the dx kernel and
    the two-stage column sums): bitwise equal, ragged chunks included; D = 1100 takes the
    separate kernels either way."""
    n, d = nd
    print(f"layernorm one pass {dtype} N={n} D={d}", flush=True)
    x = _dev(_randn((n, d), 60, 2.0) + 0.5, dtype)
    g = _dev(1.0 + 0.1 * _randn((d,), 61), dtype)
    dy = _dev(_randn((n, d), 62), dtype)
    _, mean, rstd = _capi.layernorm_fwd(x, g, torch.zeros_like(g))
    dg1, db1 = torch.zeros_like(g), torch.zeros_like(g)
    dx1 = _capi.layernorm_bwd(x, g, dy, mean, rstd, dg1, db1)
    dx2 = _capi.layernorm_bwd(x, g, dy, mean, rstd)
    dg2, db2 = torch.zeros_like(g), torch.zeros_like(g)
    lib = _capi.load()
    code = _capi._DTYPE_CODE[dtype]
    nbytes = lib.ctattn_layernorm_bwd_workspace_bytes(code, n, d)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    rc = lib.ctattn_layernorm_bwd(code, x.data_ptr(), g.data_ptr(), dy.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                                  None, dg2.data_ptr(), db2.data_ptr(), ws.data_ptr(), nbytes, n, d, None)
    assert rc == 0, _capi.last_error()
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx2) and torch.equal(dg1, dg2) and torch.equal(db1, db2)


# ---- activations ---------------------------------------------------------------------------

ACTS = {
    _capi.ACT_RELU: torch.relu,
    _capi.ACT_GELU: lambda x: F.gelu(x, approximate="tanh"),
    _capi.ACT_SIGMOID: torch.sigmoid,
    _capi.ACT_TANH: torch.tanh,
}


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("kind", sorted(ACTS))
def test_activation_fwd_bwd(dtype, kind):
    n = 10007
    x = _dev(_randn((n,), 20 + kind, 3.0), dtype)
    dy = _dev(_randn((n,), 30 + kind), dtype)
    y = _capi.activation_fwd(x, kind)
    dx = _capi.activation_bwd(x, dy, kind)
    torch.cuda.synchronize()
    x64 = _as64(x, dtype).requires_grad_(True)
    ref = ACTS[kind](x64)
    ref.backward(_as64(dy, dtype))
    tol = 4e-6 if dtype == torch.float32 else TOL[dtype]
    _close(y, ref.detach(), tol, "y")
    _close(dx, x64.grad, tol, "dx")


def test_tanh_fp32_within_4_ulp():
    """The fp32 tanh of the activations (the Maclaurin series below |x| = 0.3, 1 - 2 / (1 +
    e^(2|x|)) above) against float64 tanh on a dense grid of [-12, 12] and on magnitudes down to
    1e-8: at most 4 ulp of the float32 result (3.0 measured, at |x| just above 0.3 where the
    subtraction cancels), under 1 ulp in the series range; odd, saturating to +-1 exactly."""
    x = torch.cat([torch.linspace(-12, 12, 2_000_001), torch.logspace(-8, 0.5, 100001),
                   -torch.logspace(-8, 0.5, 100001), torch.tensor([0.0, 30.0, -30.0, 1e4, -1e4])])
    y = _capi.activation_fwd(x.to(DEV), 3).cpu()
    ref = torch.tanh(x.to(F64))
    ulp = (y.to(F64) - ref).abs() / torch.from_numpy(np.spacing(ref.abs().to(torch.float32).numpy())).to(F64)
    assert float(ulp.max()) <= 4.0, f"max {float(ulp.max()):.2f} ulp at x = {float(x[ulp.argmax()])}"
    assert float(ulp[x.abs() < 0.3].max()) <= 1.0
    assert torch.equal(y[-4:], torch.tensor([1.0, -1.0, 1.0, -1.0])) and float(y[-5]) == 0.0
    assert torch.equal(y[:1_000_000], -y[1_000_001:2_000_001].flip(0)), "tanh(-x) = -tanh(x)"


FUSED_SHAPES = [(300, 1536, 384), (4096, 384, 1536), (4096, 1024, 512), (4096, 1536, 384), (100, 96, 256),
                (37, 130, 65)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("kind", [0, 1, 2, 3], ids=["relu", "gelu", "sigmoid", "tanh"])
@pytest.mark.parametrize("mnk", FUSED_SHAPES)
def test_linear_act_fused_equals_separate(dtype, kind, mnk, gemm_path):
    """ctattn_linear_act_fwd / _bwd (the activation in the GEMM epilogue where the MFMA GEMMs
    take the shape, else the two launches) against ctattn_linear_* followed by
    ctattn_activation_*: pre, y, dpre, dw and db bitwise equal, for every activation, storage
    type and GEMM path, aligned and ragged shapes (N = 130 / K = 65: the two-step fallback;
    4096 x 1024 x 512: the 16-bit shared-tile GEMM, one- and two-chunk stages; 4096 x 1536 x 384:
    the fp32 one)."""
    m, n, k = mnk
    print(f"fused linear+act {dtype} kind={kind} M={m} N={n} K={k} policy={gemm_path}", flush=True)
    x = _dev(_randn((m, k), 80 + kind), dtype)
    w = _dev(_randn((n, k), 81, 1.0 / math.sqrt(k)), dtype)
    b = _dev(_randn((n,), 82), dtype)
    pre, y = _capi.linear_act_fwd(x, w, b, kind)
    pre_ref = _capi.linear_fwd(x, w, b)
    y_ref = _capi.activation_fwd(pre_ref, kind)
    torch.cuda.synchronize()
    assert torch.equal(pre, pre_ref) and torch.equal(y, y_ref)
    # Backward of act -> linear(w2): the linear layer's input is y = act(pre), its output dim n2.
    n2 = 2 * k + 32
    w2 = _dev(_randn((n2, n), 83, 1.0 / math.sqrt(n)), dtype)
    dy = _dev(_randn((m, n2), 84), dtype)
    dw, db = torch.zeros_like(w2), torch.zeros(n2, dtype=dtype, device=DEV)
    dw_ref, db_ref = torch.zeros_like(w2), torch.zeros(n2, dtype=dtype, device=DEV)
    dpre = _capi.linear_act_bwd(y, w2, dy, pre, kind, dw, db)
    dx_ref = _capi.linear_bwd(y, w2, dy, dw_ref, db_ref)
    dpre_ref = _capi.activation_bwd(pre, dx_ref, kind)
    torch.cuda.synchronize()
    assert torch.equal(dpre, dpre_ref)
    assert torch.equal(dw, dw_ref) and torch.equal(db, db_ref)


def test_activation_rejects_unknown_kind():
    x = torch.zeros(8, device=DEV)
    with pytest.raises(RuntimeError, match="unknown activation"):
        _capi.activation_fwd(x, 7)


# ---- embeddings ----------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_embedding_fwd_is_exact(dtype):
    b, t, e, vocab, max_len = 3, 50, 96, 65, 64
    ids = torch.randint(0, vocab, (b, t), generator=_gen(40), dtype=torch.int32)
    ids[0, 0], ids[1, 5], ids[2, 7] = -1, vocab, 1 << 30  # out-of-range ids read a zero row
    tok = _randn((vocab, e), 41).to(dtype)
    pos = _randn((max_len, e), 42).to(dtype)
    got = _capi.embedding_fwd(ids.to(DEV), tok.to(DEV), pos.to(DEV))
    only_tok = _capi.embedding_fwd(ids.to(DEV), tok.to(DEV), None)
    only_pos = _capi.embedding_fwd(ids.to(DEV), None, pos.to(DEV))
    torch.cuda.synchronize()
    valid = (ids >= 0) & (ids < vocab)
    # Sums of two stored values are exact in fp64 and in the fp32 the narrow kernels add in, so
    # the rounded fp64 sum is the kernel's result bit for bit.
    rows = torch.where(valid[..., None], tok.double()[ids.clamp(0, vocab - 1).long()], torch.zeros((), dtype=F64))
    ref_tok = rows
    ref_pos = pos.double()[:t].expand(b, t, e)
    assert torch.equal(only_tok.double().cpu(), ref_tok.to(dtype).double())
    assert torch.equal(only_pos.double().cpu(), ref_pos)
    assert torch.equal(got.double().cpu(), (ref_tok + ref_pos).to(dtype).double())


# Token-gradient rows collect about 8 contributions each here; every atomic add rounds to the
# storage type, so 16-bit tables are held to a few roundings of that many adds.
EMB_BWD_TOL = {torch.float32: 1e-6, torch.bfloat16: 4e-2, torch.float16: 5e-3, F64: 1e-12}


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_embedding_bwd(dtype):
    b, t, e, vocab, max_len = 4, 33, 40, 17, 40
    ids = torch.randint(0, vocab, (b, t), generator=_gen(43), dtype=torch.int32)
    ids[3, 3] = -2
    dout = _randn((b, t, e), 44)
    dtok0, dpos0 = _randn((vocab, e), 45), _randn((max_len, e), 46)
    dtok, dpos = _dev(dtok0, dtype), _dev(dpos0, dtype)
    _capi.embedding_bwd(ids.to(DEV), _dev(dout, dtype), dtok, dpos, vocab=vocab)
    torch.cuda.synchronize()
    d64 = _as64(dout, dtype)
    ref_tok = _as64(dtok0, dtype).clone()
    valid = ids.flatten() >= 0
    ref_tok.index_add_(0, ids.flatten()[valid].long(), d64.reshape(-1, e)[valid])
    ref_pos = _as64(dpos0, dtype).clone()
    ref_pos[:t] += d64.sum(0)
    _close(dtok, ref_tok, EMB_BWD_TOL[dtype], "dtok")
    _close(dpos, ref_pos, max(EMB_BWD_TOL[dtype], TOL[dtype]), "dpos")
    assert torch.equal(dpos[t:].cpu(), _dev(dpos0, dtype)[t:].cpu())  # rows past T untouched


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_embedding_bwd_16bit_needs_even_width(dtype):
    ids = torch.zeros((1, 2), dtype=torch.int32, device=DEV)
    dout = torch.zeros((1, 2, 5), dtype=dtype, device=DEV)
    with pytest.raises(RuntimeError, match="even embedding width"):
        _capi.embedding_bwd(ids, dout, torch.zeros((3, 5), dtype=dtype, device=DEV), None)


def test_embedding_rejects_long_sequence():
    ids = torch.zeros((1, 9), dtype=torch.int32, device=DEV)
    tab = torch.zeros((8, 4), device=DEV)
    with pytest.raises(RuntimeError, match="invalid sizes"):
        _capi.embedding_fwd(ids, tab, tab)


# ---- softmax / cross-entropy ---------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("nv", [(1, 1), (37, 65), (4, 50257)])
@pytest.mark.parametrize("temp", [1.0, 0.7])
def test_softmax_fwd_bwd(dtype, nv, temp):
    n, v = nv
    z = _dev(_randn((n, v), 50, 4.0), dtype)
    dp = _dev(_randn((n, v), 51), dtype)
    p = _capi.softmax_fwd(z, temp)
    dz = _capi.softmax_bwd(p, dp, temp)
    torch.cuda.synchronize()
    z64 = _as64(z, dtype).requires_grad_(True)
    ref = torch.softmax(z64 / temp, -1)
    ref.backward(_as64(dp, dtype))
    tol = {torch.float32: 1e-5, F64: 1e-12}.get(dtype, TOL[dtype])
    _close(p, ref.detach(), tol, "p")
    sum_atol = {torch.float32: 1e-5, F64: 1e-12}.get(dtype, 2e-2)
    assert torch.allclose(p.double().sum(-1).cpu(), torch.ones(n, dtype=F64), atol=sum_atol)
    # The backward works from the forward's p; compare with the autograd gradient at z.
    _close(dz, z64.grad, tol * 4, "dz")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_cross_entropy_and_fused_backward(dtype):
    n, v, temp = 300, 65, 0.8
    # fp16 keeps the probabilities clear of its subnormal range (smaller logit spread).
    z = _randn((n, v), 60, 1.0 if dtype == torch.float16 else 2.0)
    tgt = torch.randint(0, v, (n,), generator=_gen(61), dtype=torch.int32)
    tgt[5], tgt[77] = -1, v  # outside [0, V): zero loss, zero gradient
    p = _dev(torch.softmax(z / temp, -1), dtype)
    loss = _capi.cross_entropy_fwd(p, tgt.to(DEV))
    dp = _capi.cross_entropy_bwd(p, tgt.to(DEV))
    dz = _capi.softmax_cross_entropy_bwd(p, tgt.to(DEV), temp)
    torch.cuda.synchronize()
    p64 = _as64(p, dtype)
    valid = (tgt >= 0) & (tgt < v)
    safe = tgt.clamp(0, v - 1).long()
    ref_loss = torch.where(valid, -torch.log(p64.gather(1, safe[:, None])[:, 0]) / n, torch.zeros((), dtype=F64))
    assert loss.dtype == _capi._stat_dtype(dtype)
    _close(loss, ref_loss, 1e-12 if dtype == F64 else 1e-6, "loss")
    onehot = F.one_hot(safe, v).to(F64) * valid[:, None]
    ref_dp = torch.where(onehot > 0, -1.0 / (p64 * n), torch.zeros((), dtype=F64))
    _close(dp, ref_dp, TOL[dtype], "dp")
    # dz is the gradient of the mean cross-entropy of softmax(l / T) with respect to logits l
    # whose softmax is the p the kernel saw: l = T log p (invalid rows contribute nothing).
    logits = (temp * torch.log(p64)).requires_grad_(True)
    lp = torch.log_softmax(logits / temp, -1)
    (-(lp.gather(1, safe[:, None])[:, 0] * valid).sum() / n).backward()
    _close(dz, logits.grad, TOL[dtype] * 2, "dz")
    assert float(dz[5].abs().max()) == 0.0 and float(dz[77].abs().max()) == 0.0


# ---- Adam / AdamW --------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, F64], ids=["f32", "f64"])
@pytest.mark.parametrize("decoupled", [False, True])
def test_adam_matches_torch(dtype, decoupled):
    n, lr, wd = 5000, 1e-2, 0.05
    p0 = _randn((n,), 70)
    grads = [_randn((n,), 71 + s) for s in range(4)]
    p = _dev(p0, dtype)
    m = torch.zeros(n, device=DEV, dtype=_capi._stat_dtype(dtype))
    v = torch.zeros(n, device=DEV, dtype=_capi._stat_dtype(dtype))
    ref = _as64(p0, dtype).clone().requires_grad_(True)
    opt_cls = torch.optim.AdamW if decoupled else torch.optim.Adam
    opt = opt_cls([ref], lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    for step, g in enumerate(grads, start=1):
        _capi.adam_update(p, _dev(g, dtype), m, v, step, lr=lr, weight_decay=wd, decoupled=decoupled)
        ref.grad = _as64(g, dtype)
        opt.step()
    torch.cuda.synchronize()
    assert float((p.double().cpu() - ref.detach()).abs().max()) <= (2e-6 if dtype == torch.float32 else 1e-13)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_adam_16bit_rounds_one_fp32_update(dtype):
    """16-bit parameters: fp32 moments and arithmetic, the parameter rounded once per step."""
    n, lr, wd = 3000, 1e-2, 0.05
    p = _dev(_randn((n,), 72), dtype)
    g = _dev(_randn((n,), 73), dtype)
    p64, g64 = _as64(p, dtype), _as64(g, dtype)
    m = torch.zeros(n, device=DEV)
    v = torch.zeros(n, device=DEV)
    _capi.adam_update(p, g, m, v, 1, lr=lr, weight_decay=wd)
    torch.cuda.synchronize()
    # The kernel holds the betas in fp32 (their bias corrections come from the exact betas).
    b1, b2 = float(torch.tensor(0.9, dtype=torch.float32)), float(torch.tensor(0.999, dtype=torch.float32))
    gd = g64 + wd * p64
    m1, v1 = (1 - b1) * gd, (1 - b2) * gd * gd
    ref = p64 - lr * (m1 / 0.1) / (torch.sqrt(v1 / 0.001) + 1e-8)
    _close(m, m1, 1e-6, "m")
    _close(v, v1, 1e-6, "v")
    # one rounding of the fp32 result to the storage type: within one ulp of the exact update
    ulp = ref.abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)
    assert bool(((p.double().cpu() - ref).abs() <= ulp + 1e-30).all())


def test_adam_rejects_step_zero():
    t = torch.zeros(4, device=DEV)
    with pytest.raises(RuntimeError, match="step >= 1"):
        _capi.adam_update(t, t, t.clone(), t.clone(), 0)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_adam_multi_matches_single_bitwise(dtype):
    """One launch per 32 tensors gives exactly the per-tensor update (same arithmetic)."""
    sizes = [1, 3, 4096, 4097, 70000] + [5 + 13 * i for i in range(35)]  # 40 tensors: two launches
    ps = [_dev(_randn((n,), 80 + i), dtype) for i, n in enumerate(sizes)]
    gs = [_dev(_randn((n,), 180 + i), dtype) for i, n in enumerate(sizes)]
    ms = [torch.zeros(n, device=DEV, dtype=_capi._stat_dtype(dtype)) for n in sizes]
    vs = [torch.zeros(n, device=DEV, dtype=_capi._stat_dtype(dtype)) for n in sizes]
    ref = [(p.clone(), m.clone(), v.clone()) for p, m, v in zip(ps, ms, vs)]
    for decoupled in (False, True):
        for step in (1, 2):
            _capi.adam_update_multi(ps, gs, ms, vs, step, lr=3e-3, weight_decay=0.01, decoupled=decoupled)
            for (p, m, v), g in zip(ref, gs):
                _capi.adam_update(p, g, m, v, step, lr=3e-3, weight_decay=0.01, decoupled=decoupled)
    torch.cuda.synchronize()
    for (p, m, v), p2, m2, v2 in zip(ref, ps, ms, vs):
        assert torch.equal(p, p2) and torch.equal(m, m2) and torch.equal(v, v2)


def test_adam_multi_misaligned_views_match_single():
    """fp32 tensors whose bases are not 16-byte aligned (views one element into a buffer, some
    of the four per tensor only) take the element-wise path of the multi-tensor launch and
    still equal the per-tensor update bitwise."""
    sizes = [4096, 4099, 9000, 17]
    def view(n, seed, off):
        return _dev(_randn((n + 1,), seed), torch.float32)[off:off + n]
    ps = [view(n, 300 + i, i % 2) for i, n in enumerate(sizes)]
    gs = [view(n, 400 + i, 1) for i, n in enumerate(sizes)]
    ms = [torch.zeros(n + 1, device=DEV)[(i + 1) % 2:(i + 1) % 2 + n] for i, n in enumerate(sizes)]
    vs = [torch.zeros(n + 1, device=DEV)[:n] for n in sizes]
    ref = [(p.clone(), m.clone(), v.clone()) for p, m, v in zip(ps, ms, vs)]
    for step in (1, 2):
        _capi.adam_update_multi(ps, gs, ms, vs, step, lr=3e-3, weight_decay=0.01, decoupled=True)
        for (p, m, v), g in zip(ref, gs):
            _capi.adam_update(p, g, m, v, step, lr=3e-3, weight_decay=0.01, decoupled=True)
    torch.cuda.synchronize()
    for (p, m, v), p2, m2, v2 in zip(ref, ps, ms, vs):
        assert torch.equal(p, p2) and torch.equal(m, m2) and torch.equal(v, v2)


def test_zero_multi_clears_exactly_the_given_bytes():
    arena = torch.full((1 << 16,), 0xAB, dtype=torch.uint8, device=DEV)
    spans = [(0, 4), (16, 7), (64, 4096 * 4 + 3), (40000, 1)] + [(50000 + 64 * i, 12) for i in range(34)]
    views = [arena[o:o + n] for o, n in spans]
    _capi.zero_multi(views)
    torch.cuda.synchronize()
    expect = torch.full_like(arena, 0xAB).cpu()
    for o, n in spans:
        expect[o:o + n] = 0
    assert torch.equal(arena.cpu(), expect)


# ---- mean squared error --------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("shape", [(1, 1), (37, 65), (3, 5, 130)])
def test_mse_loss(dtype, shape):
    x = _dev(_randn(shape, 90), dtype)
    y = _dev(_randn(shape, 91), dtype)
    loss = _capi.mse_loss_fwd(x, y)
    dx = _capi.mse_loss_bwd(x, y)
    torch.cuda.synchronize()
    x64 = _as64(x, dtype).requires_grad_(True)
    ref = ((x64 - _as64(y, dtype)) ** 2).mean(-1)
    ref.sum().backward()
    assert loss.shape == shape[:-1] and loss.dtype == _capi._stat_dtype(dtype)
    _close(loss, ref.detach(), _stat_tol(dtype), "loss")
    _close(dx, x64.grad, TOL[dtype], "dx")
