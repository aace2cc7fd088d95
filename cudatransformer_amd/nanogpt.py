"""NanoGPT in torch with its attention on the MI355X kernels.

Two roles: the torch-hosted training step (torch supplies the layers around attention), and,
with ``attention="sdpa"`` in float64 on the CPU, the reference that the fully native model
``cuda_transformer.FloatNanoGPT`` (every layer in libctattn.so) is checked against.  The
architecture follows the reference's NanoGPT
(``NanoGPT.cu:83-94``: token + position embedding -> Transformer -> un-embedding ->
softmax; ``TransformerBlockLayer.cu:60-66``: LayerNorm -> Attention -> LayerNorm -> MLP
with **no residual connections**; ``AttentionLayer.cu:75-102``: QKV projection with bias ->
flash attention -> output projection with bias; ``MLPLayer`` Linear -> activation (GELU in
its tanh approximation by default, ``gelu_kernels.cu:31-50``; ReLU / Sigmoid / Tanh) ->
Linear; ``Embedding.cu:314-360``:
un-embedding without bias; LayerNorm epsilon 1e-5, ``LayerNorm.cu:31``), while torch
supplies the surrounding layers and Adam.  Attention itself (forward and backward) runs in
libctattn.so through ``cudatransformer_amd.flash_attention``; with ``attention="sdpa"`` the
same module uses torch's SDPA instead, which is how the fp64 CPU reference of a training
step is built in the tests.

Deliberate departures from the reference: causal attention (config 5), textbook Adam
(the reference increments its step twice, ``AdamOptimizer.cu:75,95``), mean cross-entropy
over all tokens on logits (mathematically -log softmax), weights initialised N(0, 0.02^2)
(the reference initialises every weight to zero, ``LinearLayer.cu:28``).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._capi import flash_attention

CONFIG5 = dict(vocab=65, max_seq_len=256, d_model=384, n_heads=6, head_dim=64, mlp_dim=1536,
               n_layers=6, batch=16, seq_len=256, lr=3e-4)


# MLP activations of the reference's ActivationType (gelu: tanh approximation).
_ACTIVATIONS = {
    "relu": F.relu,
    "gelu": lambda x: F.gelu(x, approximate="tanh"),
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
}


class Attention(nn.Module):
    """QKV projection -> attention core -> output projection (AttentionLayer.cu:75-102)."""

    def __init__(self, d_model, n_heads, head_dim, causal, attention):
        super().__init__()
        self.n_heads, self.head_dim, self.causal, self.attention = n_heads, head_dim, causal, attention
        inner = n_heads * head_dim
        self.q = nn.Linear(d_model, inner)
        self.k = nn.Linear(d_model, inner)
        self.v = nn.Linear(d_model, inner)
        self.o = nn.Linear(inner, d_model)

    def forward(self, x):
        b, t, _ = x.shape
        # [B, T, H*d] -> [B, H, T, d]: the layout attention_qkv_kernels.cu:112-120 writes.
        split = lambda y: y.view(b, t, self.n_heads, self.head_dim).transpose(1, 2).contiguous()  # noqa: E731
        q, k, v = split(self.q(x)), split(self.k(x)), split(self.v(x))
        if self.attention == "ctattn":
            o = flash_attention(q, k, v, self.causal)
        else:
            o = F.scaled_dot_product_attention(q, k, v, is_causal=self.causal)
        return self.o(o.transpose(1, 2).reshape(b, t, self.n_heads * self.head_dim))


class Block(nn.Module):
    """LayerNorm -> Attention -> LayerNorm -> MLP, no residuals (TransformerBlockLayer.cu:60-66)."""

    def __init__(self, d_model, n_heads, head_dim, mlp_dim, causal, attention, activation="gelu"):
        super().__init__()
        if activation not in _ACTIVATIONS:
            raise ValueError(f"activation must be one of {sorted(_ACTIVATIONS)}")
        self.act = _ACTIVATIONS[activation]
        self.ln1 = nn.LayerNorm(d_model, eps=1e-5)
        self.attn = Attention(d_model, n_heads, head_dim, causal, attention)
        self.ln2 = nn.LayerNorm(d_model, eps=1e-5)
        self.fc1 = nn.Linear(d_model, mlp_dim)
        self.fc2 = nn.Linear(mlp_dim, d_model)

    def forward(self, x):
        x = self.attn(self.ln1(x))
        return self.fc2(self.act(self.fc1(self.ln2(x))))


class NanoGPT(nn.Module):
    def __init__(self, vocab, max_seq_len, d_model, n_heads, head_dim, mlp_dim, n_layers,
                 causal=True, attention="ctattn", activation="gelu", **_):
        super().__init__()
        if attention not in ("ctattn", "sdpa"):
            raise ValueError("attention must be 'ctattn' or 'sdpa'")
        self.config = dict(vocab=vocab, max_seq_len=max_seq_len, d_model=d_model, n_heads=n_heads,
                           head_dim=head_dim, mlp_dim=mlp_dim, n_layers=n_layers, causal=causal,
                           activation=activation)
        self.tok = nn.Embedding(vocab, d_model)
        self.pos = nn.Embedding(max_seq_len, d_model)
        self.blocks = nn.ModuleList(
            Block(d_model, n_heads, head_dim, mlp_dim, causal, attention, activation) for _ in range(n_layers))
        self.unembed = nn.Linear(d_model, vocab, bias=False)

    def init_weights(self, seed: int):
        """Weights N(0, 0.02^2), biases 0, LayerNorm (1, 0), from a seeded CPU generator so the
        GPU model and its CPU reference start identical."""
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for name, p in self.named_parameters():
                if name.endswith("bias"):
                    p.zero_()
                elif ".ln" in name:
                    p.fill_(1.0)
                else:
                    p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float64).to(p.dtype) * 0.02)
        return self

    def forward(self, ids):
        t = ids.shape[1]
        x = self.tok(ids) + self.pos(torch.arange(t, device=ids.device))
        for blk in self.blocks:
            x = blk(x)
        return self.unembed(x)

    def loss(self, ids, targets):
        logits = self.forward(ids)
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1))


_NATIVE_PARTS = {
    ("ln1",): "firstNorm", ("ln2",): "secondNorm",
    ("attn", "q"): "attention.query", ("attn", "k"): "attention.key",
    ("attn", "v"): "attention.value", ("attn", "o"): "attention.output",
    ("fc1",): "mlp.layer_0", ("fc2",): "mlp.layer_2",
}
_NATIVE_FIXED = {"tok.weight": "tokenEmbedding", "pos.weight": "positionEmbedding", "unembed.weight": "unEmbedding"}


def native_parameter_name(name: str, checkpoint_gap: int = 0) -> str:
    """Name of a parameter of this module in the native model's (and the reference's)
    parameter map: "tokenEmbedding", "positionEmbedding", "unEmbedding" and
    "layer_<slot>.<sub-layer>.<weights|biases>" (TransformerLayer.cu:167-215,
    TransformerBlockLayer.cu:119-145, MLPLayer.cu:105-118), where slot counts the
    CheckpointLayer the reference inserts before every checkpoint_gap-th block."""
    if name in _NATIVE_FIXED:
        return _NATIVE_FIXED[name]
    _, i, *rest = name.split(".")
    i = int(i)
    slot = i + (i // checkpoint_gap if checkpoint_gap else 0)
    leaf = {"weight": "weights", "bias": "biases"}[rest[-1]]
    return f"layer_{slot}.{_NATIVE_PARTS[tuple(rest[:-1])]}.{leaf}"


_NATIVE_ACT = {"relu": "ReLU", "gelu": "GELU", "sigmoid": "Sigmoid", "tanh": "Tanh"}


def to_native(model: "NanoGPT", checkpoint_gap: int = 0, temperature: float = 1.0, dtype: str = "Float"):
    """A cuda_transformer.<dtype>NanoGPT (dtype "Float", "BFloat", "Half" or "Double") with this
    module's configuration and weights (rounded to the dtype)."""
    from . import cuda_transformer as ctm

    c = model.config
    tensor = getattr(ctm, f"{dtype}Tensor")
    nat = getattr(ctm, f"{dtype}NanoGPT")(c["vocab"], c["max_seq_len"], c["d_model"], c["n_heads"], c["head_dim"], c["mlp_dim"],
                           c["n_layers"], checkpoint_gap=checkpoint_gap, temperature=temperature,
                           activation_type=getattr(ctm.ActivationType, _NATIVE_ACT[c["activation"]]),
                           causal=c["causal"])
    nat.setParameters({native_parameter_name(n, checkpoint_gap):
                       tensor.fromNumpy(p.detach().double().cpu().numpy())
                       for n, p in model.named_parameters()})
    return nat


def make_batch(batch, seq_len, vocab, seed: int):
    """Uniform random token ids and next-token targets (seed 5)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (batch, seq_len + 1), generator=g)
    return ids[:, :-1].contiguous(), ids[:, 1:].contiguous()


def train_step(model, opt, ids, targets):
    opt.zero_grad(set_to_none=True)
    loss = model.loss(ids, targets)
    loss.backward()
    opt.step()
    return loss.detach()


def attention_flops_per_step(cfg=CONFIG5) -> float:
    """Algorithmic attention flops of one fwd+bwd step (FA2 convention, causal half)."""
    fwd = 4.0 * cfg["batch"] * cfg["n_heads"] * cfg["seq_len"] ** 2 * cfg["head_dim"] / 2.0
    return 3.5 * fwd * cfg["n_layers"]


def model_flops_per_step(cfg=CONFIG5) -> float:
    """Dense matmul flops of one fwd+bwd step (3x forward) plus attention."""
    n = cfg["batch"] * cfg["seq_len"]
    e, m, inner = cfg["d_model"], cfg["mlp_dim"], cfg["n_heads"] * cfg["head_dim"]
    per_layer = 2 * n * (3 * e * inner + inner * e + 2 * e * m)
    dense = 3 * (cfg["n_layers"] * per_layer + 2 * n * e * cfg["vocab"])
    return dense + attention_flops_per_step(cfg)


__all__ = ["CONFIG5", "NanoGPT", "make_batch", "train_step", "attention_flops_per_step",
           "model_flops_per_step"]
