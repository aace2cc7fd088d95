"""NanoGPT (config 5) training step with attention on the ctattn kernels.

The fp64 CPU reference is the same module with torch SDPA as its attention; on the GPU the
attention forward and backward run in libctattn.so.
"""
import copy

import pytest
import torch

from cudatransformer_amd.nanogpt import CONFIG5, NanoGPT, make_batch, train_step

TINY = dict(vocab=17, max_seq_len=32, d_model=32, n_heads=2, head_dim=16, mlp_dim=64, n_layers=2)


def test_cpu_reference_trains():
    torch.manual_seed(0)
    model = NanoGPT(**TINY, attention="sdpa").double().init_weights(1)
    ids, tgt = make_batch(4, 32, TINY["vocab"], seed=5)
    opt = torch.optim.Adam(model.parameters(), lr=3e-3)
    losses = [float(train_step(model, opt, ids, tgt)) for _ in range(15)]
    assert abs(losses[0] - torch.log(torch.tensor(17.0)).item()) < 0.1
    assert losses[-1] < losses[0] - 0.1


def test_init_is_deterministic():
    a = NanoGPT(**TINY, attention="sdpa").init_weights(3)
    b = NanoGPT(**TINY, attention="sdpa").init_weights(3)
    for (na, pa), (nb, pb) in zip(a.named_parameters(), b.named_parameters()):
        assert na == nb and torch.equal(pa, pb)


def test_unknown_attention_rejected():
    with pytest.raises(ValueError):
        NanoGPT(**TINY, attention="naive")


@pytest.mark.gpu
def test_config5_step_matches_fp64_reference():
    """One config-5 step: loss and every parameter gradient against the fp64 CPU model."""
    cfg = CONFIG5
    gpu = NanoGPT(**cfg, attention="ctattn").init_weights(7).cuda()
    ref = NanoGPT(**cfg, attention="sdpa").init_weights(7).double()
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=5)
    loss_g = gpu.loss(ids.cuda(), tgt.cuda())
    loss_g.backward()
    loss_r = ref.loss(ids, tgt)
    loss_r.backward()
    assert abs(loss_g.item() - loss_r.item()) <= 1e-5 * abs(loss_r.item())
    for (n, pg), (_, pr) in zip(gpu.named_parameters(), ref.named_parameters()):
        g, r = pg.grad.double().cpu(), pr.grad
        scale = float(r.abs().max())
        assert float((g - r).abs().max()) <= 1e-3 * scale + 1e-9, n


@pytest.mark.gpu
def test_config5_trains_end_to_end():
    cfg = CONFIG5
    model = NanoGPT(**cfg, attention="ctattn").init_weights(11).cuda()
    opt = torch.optim.Adam(model.parameters(), lr=cfg["lr"], betas=(0.9, 0.999), eps=1e-8)
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=5)
    ids, tgt = ids.cuda(), tgt.cuda()
    losses = [float(train_step(model, opt, ids, tgt)) for _ in range(20)]
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0] - 0.05, losses
