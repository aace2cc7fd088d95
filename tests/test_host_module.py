"""The C++ host module `cuda_transformer` (Tensor / FlashAttentionLayer over the C-ABI).

CPU tests: the module imports and exposes the reference-shaped API; configuration errors
raise ValueError; without a GPU, device work raises RuntimeError (hipErrorNoDevice) instead
of crashing.  GPU tests: computeAttention / computeBackward against the fp64 oracle, the
cached and recomputed backward paths, bf16, and error translation.
"""
import numpy as np
import pytest
import torch

import cudatransformer_amd  # noqa: F401  (imports torch first, then the native libraries)
from cudatransformer_amd import cuda_transformer as ctm
from oracle import attention_fp64 as ora


def test_api_surface():
    for name in ("FloatTensor", "BFloatTensor", "FloatFlashAttentionLayer", "BFloatFlashAttentionLayer",
                 "FlashAttention", "FlashAttentionFloat", "FlashAttentionBFloat", "synchronize",
                 "set_policy", "version"):
        assert hasattr(ctm, name), name
    assert ctm.version() == 200
    layer = ctm.FloatFlashAttentionLayer(64, 12)
    assert (layer.headDim, layer.numHeads, layer.causal) == (64, 12, False)
    layer.causal = True
    assert layer.clone().causal is True
    assert not layer.hasCache()
    assert ctm.FlashAttentionBFloat(head_dim=128, num_heads=32, causal=True).causal


def test_bad_configuration_raises_value_error():
    with pytest.raises(ValueError):
        ctm.FloatFlashAttentionLayer(0, 4)
    with pytest.raises(ValueError):
        ctm.FloatFlashAttentionLayer(300, 4)
    with pytest.raises(ValueError):
        ctm.FloatFlashAttentionLayer(64, 0)


def test_no_gpu_raises_runtime_error():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError):
        ctm.FloatTensor.fromNumpy(np.zeros((1, 2, 8, 64), np.float32))


def _tensors(cls, *arrays):
    return [cls.fromNumpy(a) for a in arrays]


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_states", [True, False])
def test_float_layer_matches_oracle(causal, save_states):
    shape = (2, 4, 200, 64)
    q, k, v, do = ora.make_inputs(shape, seed=51)
    layer = ctm.FlashAttention(64, 4, causal)
    tq, tk, tv, tdo = _tensors(ctm.FloatTensor, q, k, v, do)
    o = layer.computeAttention(tq, tk, tv, save_states)
    assert layer.hasCache() == save_states
    dq, dk, dv = layer.computeBackward(tq, tk, tv, tdo)
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    got = {"o": o.numpy(), "dq": dq.numpy(), "dk": dk.numpy(), "dv": dv.numpy()}
    for key, val in got.items():
        assert val.shape == shape
        assert np.max(np.abs(val - want[key])) <= 1e-4, key
    layer.clearCache()
    assert not layer.hasCache()


@pytest.mark.gpu
@pytest.mark.parametrize("head_dim", [40, 80, 96])
def test_float_layer_padded_head_dims(head_dim):
    """Head dims without their own MFMA kernel run padded on the next width; through the C++
    layer (which sizes the backward workspace with ctattn_bwd_workspace_bytes) as through the
    C-ABI."""
    shape = (2, 3, 130, head_dim)
    q, k, v, do = ora.make_inputs(shape, seed=53 + head_dim)
    layer = ctm.FlashAttention(head_dim, 3, True)
    tq, tk, tv, tdo = _tensors(ctm.FloatTensor, q, k, v, do)
    o = layer.computeAttention(tq, tk, tv, True)
    dq, dk, dv = layer.computeBackward(tq, tk, tv, tdo)
    want = ora.attention_fwd_bwd(q, k, v, do, True)
    for key, val in {"o": o.numpy(), "dq": dq.numpy(), "dk": dk.numpy(), "dv": dv.numpy()}.items():
        assert val.shape == shape
        assert np.max(np.abs(val - want[key])) <= 1e-4, key


@pytest.mark.gpu
def test_bfloat_layer_matches_oracle():
    shape = (1, 2, 150, 64)
    q, k, v, do = ora.make_inputs(shape, seed=52, std=0.5, dtype="bf16")
    layer = ctm.FlashAttentionBFloat(64, 2, True)
    tq, tk, tv, tdo = _tensors(ctm.BFloatTensor, q, k, v, do)
    o = layer.computeAttention(tq, tk, tv, True)
    dq, dk, dv = layer.computeBackward(tq, tk, tv, tdo)
    want = ora.attention_fwd_bwd(q, k, v, do, True)
    for key, t in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        val = t.numpy()
        assert np.max(np.abs(val - want[key])) / np.max(np.abs(want[key])) <= 2e-2, key


@pytest.mark.gpu
def test_cache_is_ignored_when_shape_changes():
    layer = ctm.FlashAttention(32, 2, True)
    a = ora.make_inputs((1, 2, 64, 32), seed=53)
    b = ora.make_inputs((1, 2, 96, 32), seed=54)
    ta = _tensors(ctm.FloatTensor, *a)
    tb = _tensors(ctm.FloatTensor, *b)
    layer.computeAttention(ta[0], ta[1], ta[2], True)
    dq, dk, dv = layer.computeBackward(tb[0], tb[1], tb[2], tb[3])  # must recompute for b
    want = ora.attention_fwd_bwd(*b, True)
    assert np.max(np.abs(dq.numpy() - want["dq"])) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_in_place_write_to_output_does_not_corrupt_backward(causal):
    """The cached output shares the returned O's buffer (the reference copies it,
    FlashAttentionLayer.cu:81-84).  Writing O in place before computeBackward must not change
    the gradients: the layer sees the tensor's version count move and recomputes the forward,
    so dQ / dK / dV still match the oracle of the original inputs."""
    shape = (1, 4, 130, 64)
    q, k, v, do = ora.make_inputs(shape, seed=55)
    layer = ctm.FlashAttention(64, 4, causal)
    tq, tk, tv, tdo = _tensors(ctm.FloatTensor, q, k, v, do)
    o = layer.computeAttention(tq, tk, tv, True)
    o.fill(3.0)  # in place, after the state was cached
    o.reshape([4, 130, 64]).fill(-1.0)  # through a view of the same buffer as well
    dq, dk, dv = layer.computeBackward(tq, tk, tv, tdo)
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    for key, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.max(np.abs(t.numpy() - want[key])) <= 1e-4, key
    assert np.all(o.numpy() == -1.0)  # the caller's write stands


@pytest.mark.gpu
def test_tensor_roundtrip_and_ops():
    x = np.random.default_rng(0).standard_normal((3, 4, 5)).astype(np.float32)
    t = ctm.FloatTensor.fromNumpy(x)
    assert t.shape() == [3, 4, 5] and t.size() == 60
    assert np.array_equal(t.numpy(), x)
    c = t.clone()
    t.fill(2.5)
    assert np.all(t.numpy() == 2.5) and np.array_equal(c.numpy(), x)
    assert t.reshape([60]).shape() == [60]
    z = ctm.FloatTensor([2, 3])
    assert np.all(z.numpy() == 0)
    assert ctm.FloatTensor.fromNumpy(np.array([7.0], np.float32)).item() == 7.0
    b = ctm.BFloatTensor.fromNumpy(np.array([1.0, 1.00390625, -3.140625], np.float32))
    assert np.array_equal(b.numpy(), ora.round_to_bf16(np.array([1.0, 1.00390625, -3.140625], np.float32)))


@pytest.mark.gpu
def test_shape_errors_raise_value_error():
    layer = ctm.FlashAttention(64, 4)
    q = ctm.FloatTensor([1, 4, 16, 32])  # wrong head dim
    with pytest.raises(ValueError):
        layer.computeAttention(q, q, q)
    q2 = ctm.FloatTensor([1, 4, 16, 64])
    k2 = ctm.FloatTensor([1, 4, 17, 64])
    with pytest.raises(ValueError):
        layer.computeAttention(q2, k2, k2)


def test_type_stub_covers_the_module():
    """cuda_transformer.pyi (written by the build, as the reference's Makefile runs stubgen)
    parses and declares every public class and function of the module."""
    import ast
    import os

    path = os.path.join(os.path.dirname(ctm.__file__), "cuda_transformer.pyi")
    tree = ast.parse(open(path).read())
    declared = {n.name for n in tree.body if isinstance(n, (ast.ClassDef, ast.FunctionDef))}
    public = {n for n in dir(ctm) if not n.startswith("_")}
    assert public <= declared, sorted(public - declared)
    tensor = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "FloatTensor")
    methods = {n.name for n in tensor.body if isinstance(n, ast.FunctionDef)}
    assert {"fromNumpy", "numpy", "matmul", "__add__", "sum", "transpose"} <= methods
