"""fp16 and fp64 storage: the attention kernels (fp16 / fp64 MFMA and generic), the fp16 / fp64
projection GEMMs and the Half / Double (and BFloat) classes of the host module, up to a NanoGPT training step.

fp64 runs accumulate in fp64 (LSE and delta are fp64 too), so they match the fp64 oracle to
rounding: tolerance 1e-10 relative to the largest value.  fp16 stores IEEE binary16 and
accumulates in fp32; it is compared with the oracle on the same fp16-rounded inputs at 4e-3
relative to the largest value (binary16's unit roundoff is 2^-11 = 4.9e-4, and outputs pass
through one or two fp16-rounded intermediates).
"""
import numpy as np
import pytest
import torch

import torch.nn.functional as F

from cudatransformer_amd import _capi as ct
from cudatransformer_amd import cuda_transformer as ctm
from cudatransformer_amd.nanogpt import NanoGPT, make_batch, native_parameter_name, to_native
from oracle import attention_fp64 as ora
from oracle import attention_layer_fp64 as lay

F64_REL = 1e-10
F16_REL = 4e-3
NAME = {torch.float64: "f64", torch.float16: "f16"}


def say(msg):
    print(msg, flush=True)


def rel_check(got, want, rel, what, floor=1e-30):
    """max |got - want| <= rel * max(max |want|, floor); `floor` bounds the scale of
    quantities that are zero in exact arithmetic (the key bias gradient)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if not want.size:
        return
    err = float(np.max(np.abs(got - want)))
    scale = max(float(np.max(np.abs(want))), floor)
    assert err <= rel * scale, f"{what}: max abs err {err:.3e} vs scale {scale:.3e}"


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64)).to("cuda", dtype)


def host(t):
    return t.double().cpu().numpy()


def test_half_double_api_surface():
    for name in ("HalfTensor", "DoubleTensor", "HalfModule", "DoubleModule", "HalfFlashAttentionLayer",
                 "DoubleFlashAttentionLayer", "FlashAttentionHalf", "FlashAttentionDouble",
                 "HalfAttentionLayer", "DoubleAttentionLayer", "AttentionHalf", "AttentionDouble"):
        assert hasattr(ctm, name), name
    assert issubclass(ctm.DoubleAttentionLayer, ctm.DoubleModule)
    assert issubclass(ctm.HalfAttentionLayer, ctm.HalfModule)
    layer = ctm.FlashAttentionDouble(head_dim=40, num_heads=3, causal=True)
    assert (layer.headDim, layer.numHeads, layer.causal) == (40, 3, True)


def test_lse_dtype_follows_storage():
    assert ct._stat_dtype(torch.float64) == torch.float64
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        assert ct._stat_dtype(dt) == torch.float32


ATTN_SHAPES = [
    (2, 3, 77, 64),   # ragged T, MFMA-sized head dim
    (1, 2, 130, 40),  # head dim off the MFMA set
    (1, 1, 1, 8),     # a single row
    (1, 2, 64, 128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ATTN_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["f64", "f16"])
def test_flash_attn_capi_matches_oracle(shape, causal, dtype):
    say(f"flash_attn capi shape={shape} causal={causal} dtype={dtype}")
    name = NAME[dtype]
    q, k, v, do = ora.make_inputs(shape, seed=300 + ATTN_SHAPES.index(shape), dtype=name)
    want = ora.attention_fwd_bwd(*ora.cast_inputs((q, k, v, do), name), causal)
    tq, tk, tv, tdo = (dev(a, dtype) for a in (q, k, v, do))
    o, lse = ct.flash_attn_fwd(tq, tk, tv, causal)
    assert lse.dtype == ct._stat_dtype(dtype)
    dq, dk, dv = ct.flash_attn_bwd(tq, tk, tv, o, tdo, lse, causal)
    torch.cuda.synchronize()
    rel = F64_REL if dtype == torch.float64 else F16_REL
    # dQ and dK vanish in exact arithmetic where a row sees one key (T = 1); the fp16 MFMA
    # backward (its dP accumulator starts from -delta) leaves a few ulps there, so their scale
    # falls back to 1e-4 of the dV scale, as in the native-head-dim parity tests.
    dv_scale = float(np.max(np.abs(want["dv"])))
    for key, t in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert t.dtype == (lse.dtype if key == "lse" else dtype)
        floor = 1e-4 * dv_scale if key in ("dq", "dk") else 1e-30
        rel_check(host(t), want[key], rel, f"{name} {key}", floor=floor)


@pytest.mark.gpu
def test_f16_output_is_rounded_to_nearest():
    """Generic kernel: fp16 O equals the fp64 oracle's O rounded to binary16 except where the
    fp32 accumulation lands within a few fp32 ulps of a rounding tie (at most one binary16 ulp
    away)."""
    shape = (1, 2, 96, 64)
    q, k, v, do = ora.make_inputs(shape, seed=310, dtype="f16")
    want = ora.attention_fwd(*ora.cast_inputs((q, k, v), "f16"), True)[0]
    prev = ct.set_policy(ct.POLICY_GENERIC)  # the generic kernel keeps P in fp32
    try:
        o, _ = ct.flash_attn_fwd(*(dev(a, torch.float16) for a in (q, k, v)), True)
    finally:
        ct.set_policy(prev)
    got = host(o)
    exact = ora.round_to_f16(want).astype(np.float64)
    ulp = np.abs(exact) * 2.0 ** -10 + 2.0 ** -24
    assert np.all(np.abs(got - exact) <= ulp * 1.0001)
    assert np.mean(got == exact) > 0.99


@pytest.mark.gpu
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_f16_mfma_matches_generic_and_oracle(causal, d):
    """fp16 on the fp16 MFMA kernels (P and dS rounded to fp16 as MFMA operands, fp32
    accumulation) against the generic fp16 kernels and the fp64 oracle."""
    shape = (2, 3, 300, d)
    say(f"f16 mfma vs generic causal={causal} d={d}")
    q, k, v, do = ora.make_inputs(shape, seed=350 + d, dtype="f16")
    want = ora.attention_fwd_bwd(*ora.cast_inputs((q, k, v, do), "f16"), causal)
    t = [dev(a, torch.float16) for a in (q, k, v, do)]

    def run():
        o, lse = ct.flash_attn_fwd(t[0], t[1], t[2], causal)
        dq, dk, dv = ct.flash_attn_bwd(t[0], t[1], t[2], o, t[3], lse, causal)
        torch.cuda.synchronize()
        return {"o": host(o), "lse": host(lse), "dq": host(dq), "dk": host(dk), "dv": host(dv)}

    mfma = run()
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        generic = run()
    finally:
        ct.set_policy(prev)
    for key in mfma:
        rel_check(mfma[key], want[key], F16_REL, f"mfma {key}")
        rel_check(mfma[key], generic[key], F16_REL, f"mfma vs generic {key}")
    r1 = run()
    for key in mfma:  # no atomics in the 16-bit kernels: bitwise reproducible
        assert np.array_equal(r1[key], mfma[key]), key


F64_MFMA_SHAPES = [(2, 3, 300, 32), (2, 3, 300, 64), (1, 2, 300, 128), (1, 2, 1, 64), (3, 1, 17, 128),
                   (1, 1, 513, 64)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", F64_MFMA_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_f64_mfma_matches_generic_and_oracle(shape, causal):
    """fp64 on the fp64 MFMA kernels (16x16x4 f64, every product and sum in fp64) against the
    generic fp64 kernels and the fp64 oracle: both to rounding.  Ragged T covers partial key
    and query tiles, T = 1 a single row."""
    say(f"f64 mfma vs generic shape={shape} causal={causal}")
    q, k, v, do = ora.make_inputs(shape, seed=370 + shape[2] + shape[3], dtype="f64")
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    t = [dev(a, torch.float64) for a in (q, k, v, do)]

    def run():
        o, lse = ct.flash_attn_fwd(t[0], t[1], t[2], causal)
        assert lse.dtype == torch.float64
        dq, dk, dv = ct.flash_attn_bwd(t[0], t[1], t[2], o, t[3], lse, causal)
        torch.cuda.synchronize()
        return {"o": host(o), "lse": host(lse), "dq": host(dq), "dk": host(dk), "dv": host(dv)}

    mfma = run()
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        generic = run()
    finally:
        ct.set_policy(prev)
    for key in mfma:  # floor 1: at T = 1 dQ is zero in exact arithmetic (dS = P (dP - delta) = 0)
        rel_check(mfma[key], want[key], F64_REL, f"mfma {key}", floor=1.0)
        rel_check(mfma[key], generic[key], F64_REL, f"mfma vs generic {key}", floor=1.0)
    r1 = run()
    for key in mfma:  # no atomics in the fp64 kernels: bitwise reproducible
        assert np.array_equal(r1[key], mfma[key]), key


@pytest.mark.gpu
def test_f64_mfma_full_size_c3d():
    """The c3d bench shape (B8 H12 T1024 d64, causal, fp64): the fp64 MFMA kernels against the
    generic fp64 kernels on the GPU (both fp64 throughout; the dense numpy oracle is too slow
    at this size), plus the size-independent identities sum_t dV = sum_t dO (the softmax rows
    sum to one) and sum_t dK = 0 (dS rows sum to zero)."""
    shape = (8, 12, 1024, 64)
    say("f64 mfma vs generic at c3d size")
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v, do = (torch.randn(shape, device="cuda", dtype=torch.float64, generator=g) for _ in range(4))

    def run():
        o, lse = ct.flash_attn_fwd(q, k, v, True)
        dq, dk, dv = ct.flash_attn_bwd(q, k, v, o, do, lse, True)
        torch.cuda.synchronize()
        return {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}

    mfma = run()
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        generic = run()
    finally:
        ct.set_policy(prev)
    for key in mfma:
        err = float((mfma[key] - generic[key]).abs().max())
        scale = max(float(generic[key].abs().max()), 1.0)
        assert err <= F64_REL * scale, f"{key}: {err:.3e} vs {scale:.3e}"
    dv_sum, do_sum = mfma["dv"].sum(2), do.sum(2)
    assert float((dv_sum - do_sum).abs().max()) <= 1e-9 * float(do_sum.abs().max())
    assert float(mfma["dk"].sum(2).abs().max()) <= 1e-9 * float(mfma["dk"].abs().max()) * 1024


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["f64", "f16"])
def test_flash_layer_pybind(dtype):
    name = NAME[dtype]
    say(f"flash layer pybind dtype={dtype}")
    tensor_cls = ctm.DoubleTensor if dtype == torch.float64 else ctm.HalfTensor
    factory = ctm.FlashAttentionDouble if dtype == torch.float64 else ctm.FlashAttentionHalf
    shape = (2, 3, 100, 32)
    q, k, v, do = ora.make_inputs(shape, seed=320, std=0.7, dtype=name)
    want = ora.attention_fwd_bwd(*ora.cast_inputs((q, k, v, do), name), True)
    rel = F64_REL if dtype == torch.float64 else F16_REL
    layer = factory(32, 3, True)
    tq, tk, tv, tdo = (tensor_cls.fromNumpy(a) for a in (q, k, v, do))
    for save in (True, False):
        o = layer.computeAttention(tq, tk, tv, save)
        assert layer.hasCache() == save
        dq, dk, dv = layer.computeBackward(tq, tk, tv, tdo)
        for key, t in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
            val = t.numpy()
            assert val.dtype == (np.float64 if dtype == torch.float64 else np.float32)
            rel_check(val, want[key], rel, f"{name} save={save} {key}")
        layer.clearCache()
        assert not layer.hasCache()


@pytest.mark.gpu
def test_tensor_roundtrip_half_double():
    x = np.concatenate([np.random.default_rng(1).standard_normal(1000) * 100,
                        1.0 + (np.arange(50) * 2 + 1) * 2.0 ** -11,  # binary16 ties
                        [65504.0, 6.0e-8, 1e-5, -0.0]])
    h = ctm.HalfTensor.fromNumpy(x.astype(np.float32))
    assert np.array_equal(h.numpy(), ora.round_to_f16(x.astype(np.float32)))
    d = ctm.DoubleTensor.fromNumpy(x + 1e-12)  # values fp32 cannot hold
    back = d.numpy()
    assert back.dtype == np.float64 and np.array_equal(back, x + 1e-12)
    c = d.clone()
    d.fill(0.1)
    assert np.all(d.numpy() == 0.1) and np.array_equal(c.numpy(), x + 1e-12)


# ---- projections and the whole attention layer -------------------------------------------

LAYER_SHAPES = [
    (2, 40, 12, 2, 4),      # E != H*d
    (1, 65, 10, 3, 6),      # E, d not multiples of 4
    (2, 130, 64, 4, 16),    # several GEMM tiles
    (1, 256, 256, 4, 64),   # large K: fp16 weight gradients take the split-K path
]


def oracle_layer(inp, h, d, causal):
    f = lay.layer_fwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["bq"], inp["bk"], inp["bv"], inp["wo"],
                      inp["bo"], h, d, causal)
    g = lay.layer_bwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["wo"], f, inp["dy"], causal)
    return {**f, **g}


def run_ctypes_layer(inp, h, d, causal, dtype):
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


@pytest.mark.gpu
@pytest.mark.parametrize("dims", LAYER_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["f64", "f16"])
def test_projection_layer_capi(dims, causal, dtype):
    b, t, e, h, d = dims
    name = NAME[dtype]
    say(f"layer capi dims={dims} causal={causal} dtype={dtype}")
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=330 + LAYER_SHAPES.index(dims), dtype=name)
    got = run_ctypes_layer(inp, h, d, causal, dtype)
    want = oracle_layer(inp, h, d, causal)
    if dtype == torch.float64:
        for key in ("q", "k", "v", "y", "dc", "dx", "dwq", "dwk", "dwv", "dbq", "dbk", "dbv", "dwo", "dbo"):
            rel_check(got[key], want[key], F64_REL, f"f64 {dims} {key}", floor=1.0)
        return
    for key in ("q", "k", "v", "y"):
        rel_check(got[key], want[key], F16_REL, f"f16 {dims} {key}")
    # fp16 gradients go through fp16-rounded intermediates (c, dc, dq, ...): check each product
    # against the oracle applied to the GPU's own fp16 operands.
    xr = inp["x"].astype(np.float64).reshape(b * t, e)
    dyr = inp["dy"].astype(np.float64).reshape(b * t, e)
    rel_check(got["dwo"], dyr.T @ lay.to_rows(got["c"]), F16_REL, "dwo")
    rel_check(got["dbo"], dyr.sum(0), F16_REL, "dbo")
    rel_check(got["dc"], lay.from_rows(dyr @ inp["wo"].astype(np.float64), b, h, t, d), F16_REL, "dc")
    for n in ("q", "k", "v"):
        gr = lay.to_rows(got["d" + n])
        rel_check(got["dw" + n], gr.T @ xr, F16_REL, "dw" + n)
        rel_check(got["db" + n], gr.sum(0), F16_REL, "db" + n)
    dx = sum(lay.to_rows(got["d" + n]) @ inp["w" + n].astype(np.float64) for n in ("q", "k", "v"))
    rel_check(got["dx"], dx.reshape(b, t, e), F16_REL, "dx")


def make_pybind_layer(factory, tensor_cls, inp, h, d, causal):
    layer = factory(inp["x"].shape[2], h, d, causal)
    for part, w, bname in (("Query", "wq", "bq"), ("Key", "wk", "bk"), ("Value", "wv", "bv"), ("Output", "wo", "bo")):
        getattr(layer, f"set{part}Weights")(tensor_cls.fromNumpy(inp[w]))
        getattr(layer, f"set{part}Biases")(tensor_cls.fromNumpy(inp[bname]))
    return layer


@pytest.mark.gpu
def test_attention_layer_double():
    b, t, e, h, d = 2, 90, 48, 3, 16
    say("attention layer pybind f64")
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=340, dtype="f64")
    want = oracle_layer(inp, h, d, True)
    layer = make_pybind_layer(ctm.AttentionDouble, ctm.DoubleTensor, inp, h, d, True)
    x = ctm.DoubleTensor.fromNumpy(inp["x"])
    y = layer(x)
    dx = layer.backward(x, ctm.DoubleTensor.fromNumpy(inp["dy"]))
    rel_check(y.numpy(), want["y"], F64_REL, "y")
    rel_check(dx.numpy(), want["dx"], F64_REL, "dx")
    grads = layer.getGradients()
    for key, name in (("query.weights", "dwq"), ("key.weights", "dwk"), ("value.weights", "dwv"),
                      ("output.weights", "dwo"), ("query.biases", "dbq"), ("value.biases", "dbv"),
                      ("output.biases", "dbo")):
        rel_check(grads[key].numpy(), want[name], F64_REL, key)


@pytest.mark.gpu
def test_attention_layer_half():
    b, t, e, h, d = 2, 96, 64, 2, 32
    say("attention layer pybind f16")
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=341, dtype="f16")
    want = oracle_layer(inp, h, d, True)
    layer = make_pybind_layer(ctm.AttentionHalf, ctm.HalfTensor, inp, h, d, True)
    y = layer(ctm.HalfTensor.fromNumpy(inp["x"]))
    rel_check(y.numpy(), want["y"], F16_REL, "f16 y")


# ---- layers, losses, optimizers and NanoGPT in the other dtypes --------------------------

TINY = dict(vocab=17, max_seq_len=32, d_model=32, n_heads=2, head_dim=16, mlp_dim=64, n_layers=2)


@pytest.mark.gpu
def test_double_layers_losses_optimizers():
    say("double layers")
    rng = np.random.default_rng(400)
    x = rng.standard_normal((3, 10, 24))
    dy = rng.standard_normal((3, 10, 40))
    w = rng.standard_normal((40, 24)) * 0.2
    b = rng.standard_normal(40)
    lin = ctm.LinearDouble(24, 40)
    lin.setParameters({"weights": ctm.DoubleTensor.fromNumpy(w), "biases": ctm.DoubleTensor.fromNumpy(b)})
    tx, tdy = ctm.DoubleTensor.fromNumpy(x), ctm.DoubleTensor.fromNumpy(dy)
    rel_check(lin(tx).numpy(), x @ w.T + b, F64_REL, "linear y")
    rel_check(lin.backward(tx, tdy).numpy(), dy @ w, F64_REL, "linear dx")
    g = lin.getGradients()
    rel_check(g["weights"].numpy(), dy.reshape(-1, 40).T @ x.reshape(-1, 24), F64_REL, "linear dW")
    rel_check(g["biases"].numpy(), dy.sum((0, 1)), F64_REL, "linear db")

    sgd = ctm.DoubleSGDOptimizer(lin.getParameters(), 0.1)
    sgd.step(g)
    # one fused multiply-add per element: within an fp64 ulp of the two-step numpy result
    rel_check(lin.getWeights().numpy(), w - 0.1 * g["weights"].numpy(), 1e-15, "sgd", floor=1.0)

    ty = ctm.DoubleTensor.fromNumpy(x @ w.T)
    ln = ctm.LayerNormDouble(40, 1e-5)
    x64 = torch.from_numpy(x @ w.T).requires_grad_(True)
    ref = F.layer_norm(x64, (40,), eps=1e-5)
    ref.backward(torch.from_numpy(dy))
    rel_check(ln(ty).numpy(), ref.detach().numpy(), F64_REL, "layernorm y")
    rel_check(ln.backward(ty, tdy).numpy(), x64.grad.numpy(), F64_REL, "layernorm dx")

    gelu = ctm.GELUDouble(40)
    x64 = torch.from_numpy(x @ w.T).requires_grad_(True)
    ref = F.gelu(x64, approximate="tanh")
    ref.backward(torch.from_numpy(dy))
    rel_check(gelu(ty).numpy(), ref.detach().numpy(), F64_REL, "gelu y")
    rel_check(gelu.backward(ty, tdy).numpy(), x64.grad.numpy(), F64_REL, "gelu dx")

    mse = ctm.DoubleMSELoss()
    loss = mse(ty, tdy).numpy()
    assert loss.shape == (3, 10) and loss.dtype == np.float64
    rel_check(loss, ((x @ w.T - dy) ** 2).mean(-1), F64_REL, "mse")
    rel_check(mse.backward(ty, tdy).numpy(), 2 * (x @ w.T - dy) / 40, F64_REL, "mse grad")

    ck = ctm.CheckpointDouble()
    assert isinstance(ck, ctm.DoubleCheckpointLayer)
    np.testing.assert_array_equal(ck(ty).numpy(), x @ w.T)
    np.testing.assert_array_equal(ck.backward(ty, tdy).numpy(), dy)
    ck.clear()


@pytest.mark.gpu
@pytest.mark.parametrize("suffix", ["Half", "BFloat"])
def test_narrow_layers_and_losses(suffix):
    say(f"{suffix} layers")
    tensor = getattr(ctm, f"{suffix}Tensor")
    rnd = ora.round_to_f16 if suffix == "Half" else ora.round_to_bf16
    rel = F16_REL if suffix == "Half" else 2e-2
    rng = np.random.default_rng(401)
    x = rnd(rng.standard_normal((4, 9, 48)))
    dy = rnd(rng.standard_normal((4, 9, 48)))
    tx, tdy = tensor.fromNumpy(x), tensor.fromNumpy(dy)
    ln = getattr(ctm, f"LayerNorm{suffix}")(48)
    x64 = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    ref = F.layer_norm(x64, (48,), eps=1e-5)
    ref.backward(torch.from_numpy(dy.astype(np.float64)))
    rel_check(ln(tx).numpy(), ref.detach().numpy(), rel, "layernorm y")
    rel_check(ln.backward(tx, tdy).numpy(), x64.grad.numpy(), 2 * rel, "layernorm dx")
    mse = getattr(ctm, f"{suffix}MSELoss")()
    loss = mse(tx, tdy).numpy()
    assert loss.dtype == np.float32
    rel_check(loss, ((x.astype(np.float64) - dy) ** 2).mean(-1), 1e-5, "mse")
    sm = getattr(ctm, f"{suffix}Softmax")(0.5)
    p = sm(tx).numpy()
    rel_check(p, torch.softmax(torch.from_numpy(x.astype(np.float64)) / 0.5, -1).numpy(), rel, "softmax")


@pytest.mark.gpu
@pytest.mark.parametrize("suffix", ["Double", "Half", "BFloat"])
def test_nanogpt_step_other_dtypes(suffix):
    """One forward + backward of the native NanoGPT in each dtype against the fp64 torch
    model: fp64 to rounding; 16-bit dtypes by the loss, the probabilities and the direction
    of every gradient (cosine similarity).  The 16-bit runs use weights 4x the default
    initialisation: at 0.02 the query / key gradients (about 4e-6) fall below fp16's normal
    range, which no loss-scale-free fp16 training step can resolve."""
    say(f"nanogpt {suffix}")
    ref = NanoGPT(**TINY, causal=True, activation="gelu", attention="sdpa").init_weights(7).double()
    if suffix != "Double":
        with torch.no_grad():
            for prm in ref.parameters():
                prm.mul_(4.0)
    nat = to_native(ref, dtype=suffix)
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=5)
    ids_t = ctm.IntTensor.fromNumpy(ids.numpy().astype(np.int32))
    tgt_t = ctm.IntTensor.fromNumpy(tgt.numpy().astype(np.int32))
    probs = nat.forward(ids_t)
    loss = nat.loss(probs, tgt_t).numpy()
    assert loss.dtype == (np.float64 if suffix == "Double" else np.float32)
    ref.zero_grad(set_to_none=True)
    loss_ref = ref.loss(ids, tgt)
    loss_ref.backward()
    loss_ref = float(loss_ref.detach())
    with torch.no_grad():
        p_ref = torch.softmax(ref(ids), -1).numpy()
    tol = {"Double": 1e-10, "Half": 5e-3, "BFloat": 3e-2}[suffix]
    assert abs(loss.sum() - loss_ref) <= tol * abs(loss_ref)
    assert np.abs(probs.numpy() - p_ref).max() <= tol
    nat.zeroGrad()
    nat.backward(ids_t, probs, tgt_t)
    grads = nat.getGradients()
    for n, prm in ref.named_parameters():
        g = grads[native_parameter_name(n)].numpy().astype(np.float64).ravel()
        r = prm.grad.numpy().ravel()
        if suffix == "Double":
            rel_check(g, r, 1e-9, n, floor=1e-6)  # floor: the key-bias gradient is zero in exact arithmetic
        elif np.abs(r).max() > 1e-9:  # the key-bias gradient is zero in exact arithmetic
            cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-300))
            assert cos >= (0.999 if suffix == "Half" else 0.99), (n, cos)


@pytest.mark.gpu
def test_double_adam_training_matches_torch():
    say("nanogpt double adam")
    ref = NanoGPT(**TINY, causal=True, activation="relu", attention="sdpa").init_weights(11).double()
    nat = to_native(ref, dtype="Double")
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=12)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    opt = ctm.DoubleAdamWOptimizer(nat.getParameters(), lr=3e-3, decay=0.01)
    opt_ref = torch.optim.AdamW(ref.parameters(), lr=3e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    for _ in range(6):
        probs = nat.forward(ids_np)
        loss = float(nat.loss(probs, tgt_np).numpy().sum())
        nat.zeroGrad()
        nat.backward(ids_np, probs, tgt_np)
        opt.step(nat.getGradients())
        ref.zero_grad(set_to_none=True)
        loss_ref = ref.loss(ids, tgt)
        loss_ref.backward()
        opt_ref.step()
        assert abs(loss - float(loss_ref.detach())) <= 1e-9 * abs(float(loss_ref.detach()))
    for n, prm in ref.named_parameters():
        rel_check(nat.getParameters()[native_parameter_name(n)].numpy(), prm.detach().numpy(), 1e-9, n, floor=1.0)

