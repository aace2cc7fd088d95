"""The native NanoGPT host (cuda_transformer.FloatNanoGPT and the layers under it), every layer
in libctattn.so, against the float64 torch model of cudatransformer_amd.nanogpt (torch SDPA
attention on the CPU) with the same weights.

The reference's NanoGPT (NanoGPT.cu) returns softmax probabilities from forward, per-position
losses -log p[target] / N from loss, and accumulates gradients in backward(input, probs,
target); parameter keys are "tokenEmbedding", "positionEmbedding", "unEmbedding" and
"layer_<i>.{firstNorm,attention,secondNorm,mlp}.…" (TransformerLayer.cu:167-215,
TransformerBlockLayer.cu:119-200, MLPLayer.cu:105-146).  Tolerances: losses within 1e-5
relative, gradients within 1e-3 of each tensor's largest entry (fp32 kernels vs float64).
"""
import numpy as np
import pytest
import torch

import cudatransformer_amd  # noqa: F401  (torch first, then the native libraries)
from cudatransformer_amd import cuda_transformer as ctm
from cudatransformer_amd.nanogpt import NanoGPT, make_batch, native_parameter_name, to_native

TINY = dict(vocab=17, max_seq_len=32, d_model=32, n_heads=2, head_dim=16, mlp_dim=64, n_layers=2)
ACT = {"relu": "ReLU", "gelu": "GELU", "sigmoid": "Sigmoid", "tanh": "Tanh"}


def native_key(name: str, gap: int = 0) -> str:
    return native_parameter_name(name, gap)


def test_api_surface():
    for name in ("FloatNanoGPT", "FloatAdamOptimizer", "FloatAdamWOptimizer", "FloatTokenEmbedding",
                 "FloatPositionEmbedding", "FloatUnEmbedding", "FloatSoftmax", "BFloatSoftmax",
                 "FloatCrossEntropyLoss", "IntTensor", "FloatLinearLayer", "BFloatLinearLayer",
                 "FloatLayerNormLayer", "FloatActivationLayer", "FloatMLPLayer", "FloatTransformerBlockLayer",
                 "FloatTransformerLayer", "LayerNorm", "Linear", "Activation", "ReLU", "GELU", "Sigmoid",
                 "Tanh", "MLP", "TransformerBlock", "Transformer", "TransformerFloat", "LinearBFloat"):
        assert hasattr(ctm, name), name
    assert {m.name for m in ctm.SamplingMode.__members__.values()} == {"Greedy", "Random", "Nucleus", "TopK"}
    assert {a.name for a in ctm.ActivationType.__members__.values()} == {"ReLU", "GELU", "Sigmoid", "Tanh"}
    assert issubclass(ctm.FloatTransformerLayer, ctm.FloatModule)
    assert issubclass(ctm.FloatAdamWOptimizer, ctm.FloatAdamOptimizer)


def test_native_key_mapping():
    ref = NanoGPT(**TINY, attention="sdpa")
    keys = [native_key(n) for n, _ in ref.named_parameters()]
    assert len(set(keys)) == len(keys)
    assert "layer_1.attention.output.biases" in keys and "layer_0.mlp.layer_2.weights" in keys
    assert native_key("blocks.1.ln1.weight", gap=1) == "layer_2.firstNorm.weights"


def test_no_gpu_raises_runtime_error():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError):
        ctm.FloatNanoGPT(17, 32, 32, 2, 16, 64, 2)


# ---- GPU ---------------------------------------------------------------------------------


def build_pair(seed=7, causal=True, activation="gelu", gap=0):
    ref = NanoGPT(**TINY, causal=causal, activation=activation, attention="sdpa").init_weights(seed).double()
    nat = to_native(ref, checkpoint_gap=gap)
    assert nat.activationType() == getattr(ctm.ActivationType, ACT[activation]) and nat.causal() == causal
    return ref, nat


def ref_step(ref, ids, tgt):
    ref.zero_grad(set_to_none=True)
    loss = ref.loss(ids, tgt)
    loss.backward()
    return float(loss.detach())


@pytest.mark.gpu
@pytest.mark.parametrize("causal,activation,gap,id_tensor", [(True, "gelu", 0, True), (True, "gelu", 0, False),
                                                            (False, "relu", 0, True), (True, "tanh", 1, False)])
def test_step_matches_fp64_reference(causal, activation, gap, id_tensor):
    """id_tensor: the ids go in as one IntTensor, so backward reuses the activations forward
    kept; otherwise as NumPy arrays (a new device tensor per call), so backward recomputes."""
    print(f"native nanogpt causal={causal} act={activation} gap={gap} id_tensor={id_tensor}", flush=True)
    ref, nat = build_pair(causal=causal, activation=activation, gap=gap)
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=5)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    if id_tensor:
        ids_np, tgt_np = ctm.IntTensor.fromNumpy(ids_np), ctm.IntTensor.fromNumpy(tgt_np)

    params = nat.getParameters()
    assert set(params) == {native_key(n, gap) for n, _ in ref.named_parameters()}
    probs = nat.forward(ids_np)
    assert probs.shape() == [4, 32, TINY["vocab"]]
    loss = nat.loss(probs, tgt_np)
    assert loss.shape() == [4, 32]
    loss_ref = ref_step(ref, ids, tgt)
    assert abs(loss.numpy().sum() - loss_ref) <= 1e-5 * abs(loss_ref)
    with torch.no_grad():
        p_ref = torch.softmax(ref(ids), -1)
    assert np.abs(probs.numpy() - p_ref.numpy()).max() <= 1e-5

    nat.zeroGrad()
    nat.backward(ids_np, probs, tgt_np)
    grads = nat.getGradients()
    for n, p in ref.named_parameters():
        g = grads[native_key(n, gap)].numpy().astype(np.float64)
        r = p.grad.numpy()
        assert g.shape == r.shape, n
        scale = np.abs(r).max()
        assert np.abs(g - r).max() <= 1e-3 * scale + 1e-9, n


@pytest.mark.gpu
def test_gradients_accumulate_and_zero():
    _, nat = build_pair()
    ids, tgt = make_batch(2, 16, TINY["vocab"], seed=9)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    probs = nat.forward(ids_np)
    nat.zeroGrad()
    nat.backward(ids_np, probs, tgt_np)
    once = {k: v.numpy().copy() for k, v in nat.getGradients().items()}
    nat.backward(ids_np, probs, tgt_np)
    twice = nat.getGradients()
    for k, v in once.items():
        np.testing.assert_allclose(twice[k].numpy(), 2 * v, rtol=1e-5, atol=1e-7 * max(1.0, np.abs(v).max()))
    nat.zeroGrad()
    assert all(np.abs(v.numpy()).max() == 0 for v in nat.getGradients().values())


@pytest.mark.gpu
def test_backward_without_checkpoint_recomputes():
    _, nat = build_pair(seed=3)
    ids, tgt = make_batch(2, 16, TINY["vocab"], seed=4)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    probs = nat.forward(ids_np)
    nat.zeroGrad()
    nat.backward(ids_np, probs, tgt_np)
    with_ckpt = {k: v.numpy().copy() for k, v in nat.getGradients().items()}
    nat.clear()
    nat.zeroGrad()
    nat.backward(ids_np, probs, tgt_np)
    for k, v in nat.getGradients().items():
        np.testing.assert_allclose(v.numpy(), with_ckpt[k], rtol=1e-5, atol=1e-8)


@pytest.mark.gpu
def test_kept_activations_match_recompute():
    """backward on the forward's own ids tensor (kept activations) and after clear()
    (everything recomputed from the ids) give the same gradients."""
    _, nat = build_pair(seed=8)
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=10)
    ids = ctm.IntTensor.fromNumpy(ids.numpy().astype(np.int32))
    tgt = ctm.IntTensor.fromNumpy(tgt.numpy().astype(np.int32))
    grads = []
    for drop in (False, True):
        probs = nat.forward(ids)
        if drop:
            nat.clear()
        nat.zeroGrad()
        nat.backward(ids, probs, tgt)
        grads.append({k: v.numpy().copy() for k, v in nat.getGradients().items()})
    for k, v in grads[0].items():
        np.testing.assert_allclose(grads[1][k], v, rtol=1e-5, atol=1e-6 * max(np.abs(v).max(), 1e-30), err_msg=k)


@pytest.mark.gpu
def test_sgd_update_and_clone():
    _, nat = build_pair(seed=5)
    ids, tgt = make_batch(2, 16, TINY["vocab"], seed=6)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    twin = nat.clone()
    before = {k: v.numpy().copy() for k, v in nat.getParameters().items()}
    probs = nat.forward(ids_np)
    nat.zeroGrad()
    nat.backward(ids_np, probs, tgt_np)
    grads = {k: v.numpy().copy() for k, v in nat.getGradients().items()}
    nat.sgdUpdate(0.5)
    after = nat.getParameters()
    for k, p0 in before.items():
        np.testing.assert_allclose(after[k].numpy(), p0 - 0.5 * grads[k], rtol=0, atol=1e-6, err_msg=k)
    for k, v in twin.getParameters().items():
        assert np.array_equal(v.numpy(), before[k]), k


@pytest.mark.gpu
def test_adam_training_matches_torch_and_learns():
    ref, nat = build_pair(seed=11)
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=12)
    ids_np, tgt_np = ids.numpy().astype(np.int32), tgt.numpy().astype(np.int32)
    opt = ctm.FloatAdamOptimizer(nat.getParameters(), lr=3e-3)
    opt_ref = torch.optim.Adam(ref.parameters(), lr=3e-3, betas=(0.9, 0.999), eps=1e-8)
    losses, losses_ref = [], []
    for _ in range(25):
        probs = nat.forward(ids_np)
        losses.append(float(nat.loss(probs, tgt_np).numpy().sum()))
        nat.zeroGrad()
        nat.backward(ids_np, probs, tgt_np)
        opt.step(nat.getGradients())
        losses_ref.append(ref_step(ref, ids, tgt))
        opt_ref.step()
    assert opt.getTimeStep() == 25
    assert losses[-1] < losses[0] - 0.15, losses
    np.testing.assert_allclose(losses, losses_ref, rtol=5e-3)


@pytest.mark.gpu
def test_adam_requires_every_gradient():
    _, nat = build_pair()
    params = nat.getParameters()
    opt = ctm.FloatAdamWOptimizer(params, lr=1e-3, decay=0.01)
    grads = nat.getGradients()
    del grads["unEmbedding"]
    with pytest.raises(ValueError, match="unEmbedding"):
        opt.step(grads)
    assert opt.getTimeStep() == 0


@pytest.mark.gpu
def test_generation_and_sampling():
    ref, nat = build_pair(seed=13)
    prompt = [1, 2, 3]
    out = nat.generate(prompt, 6, ctm.SamplingMode.Greedy)
    assert isinstance(out, list) and out[:3] == prompt and len(out) == 9
    seq = list(prompt)
    with torch.no_grad():
        for _ in range(6):
            logits = ref(torch.tensor([seq]))[0, -1]
            seq.append(int(torch.argmax(logits)))
    assert out == seq
    arr = nat.generate(np.array(prompt, np.int32), 2, ctm.SamplingMode.TopK, K=1)
    assert isinstance(arr, np.ndarray) and list(arr) == seq[:5]
    ten = nat.generate(ctm.IntTensor.fromNumpy(np.array(prompt, np.int32)), 2, ctm.SamplingMode.Greedy)
    assert list(ten.numpy()) == seq[:5]
    probs = nat.forward(prompt)
    assert probs.shape() == [3, TINY["vocab"]]
    greedy = nat.predict(probs, ctm.SamplingMode.Greedy)
    assert greedy == seq[3]
    assert nat.predict(probs, ctm.SamplingMode.Nucleus, P=0.999) == greedy  # nothing above P: argmax
    for mode in (ctm.SamplingMode.Random, ctm.SamplingMode.TopK, ctm.SamplingMode.Nucleus):
        assert 0 <= nat.sample(prompt, mode, K=5, P=0.01) < TINY["vocab"]
    long_prompt = list(range(TINY["vocab"])) * 3  # longer than max_seq_len: the context is cropped
    assert len(nat.generate(long_prompt, 1, ctm.SamplingMode.Greedy)) == len(long_prompt) + 1


@pytest.mark.gpu
def test_shape_errors_raise_value_error():
    _, nat = build_pair()
    with pytest.raises(ValueError, match="maxSeqLen"):
        nat.forward(np.zeros((1, TINY["max_seq_len"] + 1), np.int32))
    probs = nat.forward(np.zeros((2, 8), np.int32))
    with pytest.raises(ValueError):
        nat.backward(np.zeros((2, 8), np.int32), probs, np.zeros((2, 7), np.int32))
    with pytest.raises(ValueError):
        nat.setTemperature(0.0)


@pytest.mark.gpu
def test_layers_through_the_module_match_torch():
    torch.manual_seed(0)
    x = torch.randn(3, 10, 24, dtype=torch.float64)
    dy = torch.randn(3, 10, 40, dtype=torch.float64)
    lin = ctm.Linear(24, 40)
    w = torch.randn(40, 24, dtype=torch.float64) * 0.2
    b = torch.randn(40, dtype=torch.float64)
    lin.setParameters({"weights": ctm.FloatTensor.fromNumpy(w.numpy()), "biases": ctm.FloatTensor.fromNumpy(b.numpy())})
    tx = ctm.FloatTensor.fromNumpy(x.numpy())
    y = lin(tx).numpy()
    dx = lin.backward(tx, ctm.FloatTensor.fromNumpy(dy.numpy())).numpy()
    x32, w32, dy32 = (t.float().double() for t in (x, w, dy))
    np.testing.assert_allclose(y, (x32 @ w32.T + b.float().double()).numpy(), atol=2e-5)
    np.testing.assert_allclose(dx, (dy32 @ w32).numpy(), atol=2e-5)
    g = lin.getGradients()
    np.testing.assert_allclose(g["weights"].numpy(), (dy32.reshape(-1, 40).T @ x32.reshape(-1, 24)).numpy(),
                               atol=1e-4)
    np.testing.assert_allclose(g["biases"].numpy(), dy32.sum((0, 1)).numpy(), atol=1e-4)
    assert np.array_equal(lin.getWeights().numpy(), w.float().numpy())

    ln = ctm.LayerNorm(40)
    assert set(ln.getParameters()) == {"weights", "biases"}
    assert np.array_equal(ln.getParameters()["weights"].numpy(), np.ones(40, np.float32))
    block = ctm.TransformerBlock(40, 2, 20, 80, ctm.ActivationType.GELU, causal=True)
    keys = set(block.getParameters())
    assert "attention.query.weights" in keys and "mlp.layer_2.biases" in keys and "secondNorm.weights" in keys
    tr = ctm.Transformer(40, 2, 20, 80, 3, checkpoint_gap=2)
    assert {k.split(".")[0] for k in tr.getParameters()} == {"layer_0", "layer_1", "layer_3"}


# ---- config 5 at full size --------------------------------------------

def config5_pair(seed=5):
    from cudatransformer_amd.nanogpt import CONFIG5
    model_cfg = {k: v for k, v in CONFIG5.items() if k not in ("batch", "seq_len", "lr")}
    ref = NanoGPT(**model_cfg, causal=True, activation="gelu", attention="sdpa").init_weights(seed).double()
    return CONFIG5, ref, to_native(ref)


@pytest.mark.gpu
def test_config5_step_matches_fp64_reference():
    """NanoGPT.cu:83-94 (forward) and :357-378 (backward) on the native host at config 5 -- 6
    layers, d_model 384, 6 heads of 64, T256, B16, vocab 65, GELU, causal -- against the float64
    torch model with the same weights: loss within 1e-5 relative, every gradient within 1e-3
    of its tensor's largest entry."""
    cfg, ref, nat = config5_pair()
    print("config 5 native step vs fp64", flush=True)
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=5)
    ids_t = ctm.IntTensor.fromNumpy(ids.numpy().astype(np.int32))
    tgt_t = ctm.IntTensor.fromNumpy(tgt.numpy().astype(np.int32))
    probs = nat.forward(ids_t)
    loss = float(nat.loss(probs, tgt_t).numpy().sum())
    nat.zeroGrad()
    nat.backward(ids_t, probs, tgt_t)
    grads = nat.getGradients()
    loss_ref = ref_step(ref, ids, tgt)
    assert abs(loss - loss_ref) <= 1e-5 * abs(loss_ref), (loss, loss_ref)
    for n, p in ref.named_parameters():
        g = grads[native_key(n)].numpy().astype(np.float64)
        r = p.grad.numpy()
        assert g.shape == r.shape, n
        err, scale = np.abs(g - r).max(), np.abs(r).max()
        assert err <= 1e-3 * scale + 1e-9, f"{n}: max err {err:.3e}, max |grad| {scale:.3e}"


@pytest.mark.gpu
def test_config5_adam_steps_track_fp64_reference():
    """20 Adam steps (lr 3e-4, betas 0.9 / 0.999, eps 1e-8) of config 5 on the native host
    against torch.optim.Adam on the float64 model from the same weights: every step's loss
    within 5e-3 relative, and the loss goes down."""
    cfg, ref, nat = config5_pair(seed=6)
    print("config 5 native Adam vs fp64", flush=True)
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=7)
    ids_t = ctm.IntTensor.fromNumpy(ids.numpy().astype(np.int32))
    tgt_t = ctm.IntTensor.fromNumpy(tgt.numpy().astype(np.int32))
    opt = ctm.FloatAdamOptimizer(nat.getParameters(), lr=cfg["lr"], b1=0.9, b2=0.999, eps=1e-8)
    opt_ref = torch.optim.Adam(ref.parameters(), lr=cfg["lr"], betas=(0.9, 0.999), eps=1e-8)
    losses, losses_ref = [], []
    for _ in range(20):
        probs = nat.forward(ids_t)
        losses.append(float(nat.loss(probs, tgt_t).numpy().sum()))
        nat.zeroGrad()
        nat.backward(ids_t, probs, tgt_t)
        opt.step(nat.getGradients())
        losses_ref.append(ref_step(ref, ids, tgt))
        opt_ref.step()
    print("losses", losses[0], losses[-1], "ref", losses_ref[0], losses_ref[-1], flush=True)
    np.testing.assert_allclose(losses, losses_ref, rtol=5e-3)
    assert losses[-1] < losses[0]
