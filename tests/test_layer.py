"""The attention layer: QKV projection -> flash attention -> output projection.

CPU tests: the pybind surface the reference's test imports (test_flash_attention.py:7) and
the C-ABI argument checks of the projection entry points.  GPU tests: the projection
entry points (ctypes) and the C++ AttentionLayer (pybind) against the fp64 layer oracle in
fp32 and bf16, gradient accumulation / SGD semantics, and the reference's own test
(test_flash_attention.py:14-52) at its full configuration against torch fp32 on the GPU.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cudatransformer_amd as ct
from cudatransformer_amd import _capi
from cudatransformer_amd import cuda_transformer as ctm
from oracle import attention_layer_fp64 as lay

F32_ATOL = 1e-4
BF16_REL = 2e-2


def say(msg):
    """Names the case on stdout (flushed) before its GPU work starts."""
    print(msg, flush=True)


# ---- CPU ---------------------------------------------------------------------------------


def test_reference_import_line():
    from cudatransformer_amd.cuda_transformer import AttentionFloat, FloatAttentionLayer, FloatModule, FloatTensor  # noqa: F401

    assert issubclass(FloatAttentionLayer, FloatModule)
    assert issubclass(ctm.BFloatAttentionLayer, ctm.BFloatModule)
    for name in ("forward", "forward_caching", "backward", "backward_caching", "sgdUpdate", "zeroGrad",
                 "__call__", "getParameters", "setParameters", "getGradients", "clone"):
        assert hasattr(FloatAttentionLayer, name), name
    for part in ("Query", "Key", "Value", "Output"):
        for kind in ("Weights", "Biases"):
            assert hasattr(FloatAttentionLayer, f"get{part}{kind}")
            assert hasattr(FloatAttentionLayer, f"set{part}{kind}")
    assert callable(ctm.Attention) and callable(ctm.AttentionBFloat)


def test_projection_entry_points_validate(tmp_path):
    lib = _capi.load()
    # unknown dtype, negative size, zero dims
    assert lib.ctattn_qkv_proj_fwd(5, *([1] * 10), 1, 2, 8, 2, 4, None) == 1
    assert "dtype" in _capi.last_error()
    assert lib.ctattn_qkv_proj_fwd(0, *([1] * 10), -1, 2, 8, 2, 4, None) == 1
    assert lib.ctattn_out_proj_fwd(0, 1, 1, None, 1, 1, 2, 0, 2, 4, None) == 1
    assert lib.ctattn_qkv_proj_bwd_workspace_bytes(0, 1, 2, 8, 0, 4) == -1
    # null pointers
    assert lib.ctattn_qkv_proj_fwd(0, None, 1, 1, 1, None, None, None, 1, 1, 1, 1, 2, 8, 2, 4, None) == 1
    assert "null" in _capi.last_error()
    assert lib.ctattn_out_proj_bwd(0, 1, None, 1, 1, 1, 1, 1, 1 << 30, 1, 2, 8, 2, 4, None) == 1
    # empty problems are no-ops
    assert lib.ctattn_qkv_proj_fwd(0, *([None] * 10), 0, 16, 8, 2, 4, None) == 0
    assert lib.ctattn_out_proj_bwd(1, *([None] * 7), 0, 3, 0, 8, 2, 4, None) == 0
    assert lib.ctattn_sgd_update(0, None, None, 0.1, 0, None) == 0
    # workspace: too small is rejected before any launch
    need = lib.ctattn_qkv_proj_bwd_workspace_bytes(0, 8, 1024, 1024, 16, 64)
    assert need > 0
    rc = lib.ctattn_qkv_proj_bwd(0, *([1] * 14), 1, need - 1, 8, 1024, 1024, 16, 64, None)
    assert rc == 1 and "workspace" in _capi.last_error()
    need_o = lib.ctattn_out_proj_bwd_workspace_bytes(0, 8, 1024, 1024, 16, 64)
    rc = lib.ctattn_out_proj_bwd(0, 1, 1, 1, 1, 1, 1, 1, need_o - 1, 8, 1024, 1024, 16, 64, None)
    assert rc == 1 and "workspace" in _capi.last_error()
    # workspace is only needed for weight / bias gradients
    rc = lib.ctattn_out_proj_bwd(0, 1, 1, 1, None, None, 1, None, 0, 8, 1024, 1024, 16, 64, None)
    assert rc != 1 or "workspace" not in _capi.last_error()


# ---- GPU helpers -------------------------------------------------------------------------


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda", dtype)


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def check(got, want, dtype, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    if dtype == torch.float32:
        scale = max(1.0, float(np.max(np.abs(want)))) if want.size else 1.0
        assert err <= F32_ATOL * scale, f"{what}: max abs err {err:.3e} (scale {scale:.2f})"
    else:
        rel = err / max(float(np.max(np.abs(want))), 1e-30) if want.size else 0.0
        assert rel <= BF16_REL, f"{what}: rel err {rel:.3e}"


LAYER_SHAPES = [
    (2, 40, 12, 2, 4),      # E != H*d, > one 32-row tile
    (1, 33, 20, 2, 8),      # ragged T
    (2, 130, 64, 4, 16),    # several 128-row GEMM tiles
    (1, 65, 10, 3, 6),      # E, d not multiples of 4: scalar-load GEMM path
    (2, 100, 96, 3, 32),
    (1, 256, 256, 4, 64),   # split-K weight gradients
]


def run_ctypes_layer(inp, h, d, causal, dtype):
    """Forward + backward through the C-ABI entry points, one call each."""
    t = {k: dev(v, dtype) for k, v in inp.items()}
    q, k, v = ct.qkv_proj_fwd(t["x"], t["wq"], t["wk"], t["wv"], t["bq"], t["bk"], t["bv"], h, d)
    c, lse = ct.flash_attn_fwd(q, k, v, causal)
    y = ct.out_proj_fwd(c, t["wo"], t["bo"])
    g = {n: torch.zeros_like(t[n]) for n in ("wq", "wk", "wv", "bq", "bk", "bv", "wo", "bo")}
    dc = ct.out_proj_bwd(c, t["dy"], t["wo"], dwo=g["wo"], dbo=g["bo"])
    dq, dk, dv = ct.flash_attn_bwd(q, k, v, c, dc, lse, causal)
    dx = ct.qkv_proj_bwd(t["x"], dq, dk, dv, t["wq"], t["wk"], t["wv"], dw=(g["wq"], g["wk"], g["wv"]),
                         db=(g["bq"], g["bk"], g["bv"]))
    torch.cuda.synchronize()
    out = dict(q=q, k=k, v=v, c=c, y=y, dc=dc, dq=dq, dk=dk, dv=dv, dx=dx)
    out.update({"d" + n: gg for n, gg in g.items()})
    return {n: host(val) for n, val in out.items()}


def oracle_layer(inp, h, d, causal):
    f = lay.layer_fwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["bq"], inp["bk"], inp["bv"], inp["wo"],
                      inp["bo"], h, d, causal)
    g = lay.layer_bwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["wo"], f, inp["dy"], causal)
    return {**f, **g}


# ---- GPU: C-ABI --------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("dims", LAYER_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_projection_layer_matches_oracle(dims, causal, dtype):
    b, t, e, h, d = dims
    say(f"layer ctypes dims={dims} causal={causal} dtype={dtype}")
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=60 + LAYER_SHAPES.index(dims),
                                dtype="bf16" if dtype == torch.bfloat16 else "f32")
    got = run_ctypes_layer(inp, h, d, causal, dtype)
    want = oracle_layer(inp, h, d, causal)
    for name in ("q", "k", "v", "y", "dc", "dx", "dwq", "dwk", "dwv", "dbq", "dbk", "dbv", "dwo", "dbo"):
        if dtype == torch.bfloat16 and name not in ("q", "k", "v", "y"):
            # bf16 gradients go through bf16-rounded intermediates (c, dc, dq, ...): compare
            # each product against the oracle applied to the GPU's own bf16 inputs.
            continue
        check(got[name], want[name], dtype, f"{dims} {name}")
    if dtype == torch.bfloat16:
        # Each backward product from the GPU's actual (bf16) operands.
        xr = inp["x"].astype(np.float64).reshape(b * t, e)
        dyr = inp["dy"].astype(np.float64).reshape(b * t, e)
        check(got["dwo"], dyr.T @ lay.to_rows(got["c"]), dtype, "dwo")
        check(got["dbo"], dyr.sum(0), dtype, "dbo")
        check(got["dc"], lay.from_rows(dyr @ inp["wo"].astype(np.float64), b, h, t, d), dtype, "dc")
        for n in ("q", "k", "v"):
            gr = lay.to_rows(got["d" + n])
            check(got["dw" + n], gr.T @ xr, dtype, "dw" + n)
            check(got["db" + n], gr.sum(0), dtype, "db" + n)
        dx = sum(lay.to_rows(got["d" + n]) @ inp["w" + n].astype(np.float64) for n in ("q", "k", "v"))
        check(got["dx"], dx.reshape(b, t, e), dtype, "dx")


@pytest.mark.gpu
def test_weight_gradients_accumulate_deterministically():
    """Two backward calls add exactly twice the gradient (no atomics: bitwise 2x)."""
    b, t, e, h, d = 2, 512, 128, 4, 32
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=71)
    tt = {k: dev(v, torch.float32) for k, v in inp.items()}
    q, k, v = ct.qkv_proj_fwd(tt["x"], tt["wq"], tt["wk"], tt["wv"], tt["bq"], tt["bk"], tt["bv"], h, d)
    dws = [torch.zeros_like(tt["wq"]) for _ in range(3)]
    dbs = [torch.zeros_like(tt["bq"]) for _ in range(3)]
    dx1 = ct.qkv_proj_bwd(tt["x"], q, k, v, tt["wq"], tt["wk"], tt["wv"], dw=dws, db=dbs)
    once = [x.clone() for x in dws + dbs]
    dx2 = ct.qkv_proj_bwd(tt["x"], q, k, v, tt["wq"], tt["wk"], tt["wv"], dw=dws, db=dbs)
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx2)
    for a, b1 in zip(dws + dbs, once):
        assert torch.equal(a, 2 * b1)
    p = tt["wq"].clone()
    ct.sgd_update(p, dws[0], 0.125)
    assert torch.allclose(p, tt["wq"] - 0.125 * dws[0], atol=0, rtol=0)


# ---- GPU: C++ AttentionLayer through pybind ----------------------------------------------


def make_pybind_layer(cls_factory, tensor_cls, inp, h, d, causal):
    layer = cls_factory(inp["x"].shape[2], h, d, causal)
    for part, w, bname in (("Query", "wq", "bq"), ("Key", "wk", "bk"), ("Value", "wv", "bv"), ("Output", "wo", "bo")):
        getattr(layer, f"set{part}Weights")(tensor_cls.fromNumpy(inp[w]))
        getattr(layer, f"set{part}Biases")(tensor_cls.fromNumpy(inp[bname]))
    return layer


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("caching", [False, True], ids=["recompute", "caching"])
def test_attention_layer_pybind_matches_oracle(causal, caching):
    b, t, e, h, d = 2, 150, 96, 3, 32
    say(f"layer pybind causal={causal} caching={caching}")
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=81)
    want = oracle_layer(inp, h, d, causal)
    layer = make_pybind_layer(ctm.AttentionFloat, ctm.FloatTensor, inp, h, d, causal)
    x = ctm.FloatTensor.fromNumpy(inp["x"])
    dy = ctm.FloatTensor.fromNumpy(inp["dy"])
    if caching:
        y, states = layer.forward_caching(x)
        assert len(states) == 4 and states[0].shape() == [b, h, t, d] and states[3].shape() == [b, h, t, d]
        dx = layer.backward_caching(x, dy, states)
    else:
        y = layer(x)
        dx = layer.backward(x, dy)
    check(y.numpy(), want["y"], torch.float32, "y")
    check(dx.numpy(), want["dx"], torch.float32, "dx")
    grads = layer.getGradients()
    for key, name in (("query.weights", "dwq"), ("key.weights", "dwk"), ("value.weights", "dwv"),
                      ("output.weights", "dwo"), ("query.biases", "dbq"), ("value.biases", "dbv"),
                      ("output.biases", "dbo")):
        check(grads[key].numpy(), want[name], torch.float32, key)
    # SGD: every parameter moves by -lr * grad; zeroGrad clears.
    params_before = {k: v.numpy().copy() for k, v in layer.getParameters().items()}
    layer.sgdUpdate(0.5)
    params_after = {k: v.numpy() for k, v in layer.getParameters().items()}
    for key in params_before:
        np.testing.assert_allclose(params_after[key], params_before[key] - 0.5 * grads[key].numpy(),
                                   rtol=1e-6, atol=1e-6)
    layer.zeroGrad()
    assert all(np.all(g.numpy() == 0) for g in layer.getGradients().values())
    clone = layer.clone()
    np.testing.assert_array_equal(clone(x).numpy(), layer(x).numpy())


@pytest.mark.gpu
def test_attention_layer_bfloat():
    b, t, e, h, d = 2, 96, 64, 2, 32
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=91, dtype="bf16")
    want = oracle_layer(inp, h, d, True)
    layer = make_pybind_layer(ctm.AttentionBFloat, ctm.BFloatTensor, inp, h, d, True)
    y = layer(ctm.BFloatTensor.fromNumpy(inp["x"]))
    check(y.numpy(), want["y"], torch.bfloat16, "bf16 y")


@pytest.mark.gpu
def test_setter_size_checked():
    layer = ctm.AttentionFloat(32, 2, 8)
    with pytest.raises(ValueError):
        layer.setQueryWeights(ctm.FloatTensor.fromNumpy(np.zeros((16, 16), np.float32)))


# ---- GPU: the reference's own test at full size ------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("n", [32, 64, 128, 256, 512, 1024, 2048, 4096, 8192])
def test_reference_flash_attention_script(n):
    """test_flash_attention.py:14-52: B=8, E=1024, H=16, D=64; weights N(0,1)/sqrt(E); the
    layer's output against Q,K,V = X W^T, per-head SDPA, O = C Wo^T in torch fp32, atol 1e-4."""
    B, E, H, D = 8, 1024, 16, 64
    say(f"reference script N={n}")
    g = torch.Generator(device="cuda").manual_seed(1000 + n)
    W = [torch.randn(E, E, device="cuda", generator=g) / np.sqrt(E) for _ in range(4)]
    layer = ctm.AttentionFloat(input_dim=E, num_heads=H, head_dim=D)
    layer.setQueryWeights(ctm.FloatTensor.fromNumpy(W[0].cpu().numpy()))
    layer.setKeyWeights(ctm.FloatTensor.fromNumpy(W[1].cpu().numpy()))
    layer.setValueWeights(ctm.FloatTensor.fromNumpy(W[2].cpu().numpy()))
    layer.setOutputWeights(ctm.FloatTensor.fromNumpy(W[3].cpu().numpy()))
    X = torch.randn(B, n, E, device="cuda", generator=g)
    out = layer(ctm.FloatTensor.fromNumpy(X.cpu().numpy()))
    with torch.no_grad():
        Q, K, V = X @ W[0].T, X @ W[1].T, X @ W[2].T
        C = torch.zeros_like(Q)
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
            for c0 in range(0, E, D):
                C[:, :, c0:c0 + D] = F.scaled_dot_product_attention(
                    Q[:, :, c0:c0 + D].contiguous(), K[:, :, c0:c0 + D].contiguous(), V[:, :, c0:c0 + D].contiguous())
        O = C @ W[3].T
    assert np.allclose(O.cpu().numpy(), out.numpy(), atol=1e-4), f"Attention output mismatch for N={n}"
