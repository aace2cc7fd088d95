"""Pins the attention-layer oracle (oracle/attention_layer_fp64.py) on the CPU.

The reference's only test of this layer (test_flash_attention.py:43-52) compares its
forward with torch: Q = X Wq^T, per-head SDPA, O = C Wo^T.  Here the oracle is checked
against that same formula, against torch fp64 autograd for every gradient (an independent
library routine), against central finite differences, against a closed form, and against
planted mistakes -- the reference's own bias-gradient defect among them -- so that a
dropped term, a transposed weight or a wrong layout fails at least one check.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_layer_fp64 as lay


def torch_layer(inp, h, d, causal):
    """The layer in torch fp64 with autograd: nn.functional.linear + SDPA per head."""
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=(k != "dy")) for k, v in inp.items()}
    b, n, e = t["x"].shape

    def split(y):
        return y.view(b, n, h, d).transpose(1, 2)

    q = split(F.linear(t["x"], t["wq"], t["bq"]))
    k = split(F.linear(t["x"], t["wk"], t["bk"]))
    v = split(F.linear(t["x"], t["wv"], t["bv"]))
    c = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    y = F.linear(c.transpose(1, 2).reshape(b, n, h * d), t["wo"], t["bo"])
    (y * t["dy"]).sum().backward()
    grads = {"d" + name: t[name].grad.numpy() for name in ("x", "wq", "wk", "wv", "bq", "bk", "bv", "wo", "bo")}
    return y.detach().numpy(), grads


def run_oracle(inp, h, d, causal):
    f = lay.layer_fwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["bq"], inp["bk"], inp["bv"], inp["wo"],
                      inp["bo"], h, d, causal)
    g = lay.layer_bwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], inp["wo"], f, inp["dy"], causal)
    return f, g


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dims", [(2, 5, 12, 3, 4), (1, 33, 20, 2, 8), (2, 40, 16, 4, 4)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layer_oracle_matches_torch_autograd(dims, causal):
    b, t, e, h, d = dims
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=7)
    f, g = run_oracle(inp, h, d, causal)
    y_ref, g_ref = torch_layer(inp, h, d, causal)
    np.testing.assert_allclose(f["y"], y_ref, rtol=1e-10, atol=1e-11)
    for name, ref in g_ref.items():
        np.testing.assert_allclose(g[name], ref, rtol=1e-9, atol=1e-10, err_msg=name)


def test_reference_test_formula():
    """test_flash_attention.py:43-52: Q,K,V = X W^T (no bias), SDPA per D-wide column slice,
    O = C Wo^T -- with E = H*D as in that test."""
    b, n, e, h, d = 2, 24, 32, 4, 8
    inp = lay.make_layer_inputs(b, n, e, h, d, seed=3)
    zero_h, zero_e = np.zeros(h * d, np.float32), np.zeros(e, np.float32)
    f = lay.layer_fwd(inp["x"], inp["wq"], inp["wk"], inp["wv"], zero_h, zero_h, zero_h, inp["wo"], zero_e, h, d)
    X = torch.tensor(inp["x"], dtype=torch.float64)
    Wq, Wk, Wv, Wo = (torch.tensor(inp[k], dtype=torch.float64) for k in ("wq", "wk", "wv", "wo"))
    Q, K, V = X @ Wq.T, X @ Wk.T, X @ Wv.T
    C = torch.zeros_like(Q)
    for c0 in range(0, e, d):
        C[:, :, c0:c0 + d] = F.scaled_dot_product_attention(Q[:, :, c0:c0 + d], K[:, :, c0:c0 + d],
                                                             V[:, :, c0:c0 + d])
    O = C @ Wo.T
    np.testing.assert_allclose(f["y"], O.numpy(), rtol=1e-10, atol=1e-11)


def test_finite_differences():
    b, t, e, h, d = 1, 6, 5, 2, 3
    inp = {k: v.astype(np.float64) for k, v in lay.make_layer_inputs(b, t, e, h, d, seed=11).items()}
    f, g = run_oracle(inp, h, d, True)

    def loss(mod):
        ff = lay.layer_fwd(mod["x"], mod["wq"], mod["wk"], mod["wv"], mod["bq"], mod["bk"], mod["bv"], mod["wo"],
                           mod["bo"], h, d, True)
        return float(np.sum(ff["y"] * inp["dy"]))

    rng = np.random.default_rng(0)
    eps = 1e-6
    for name in ("x", "wq", "wk", "wv", "bq", "bv", "wo", "bo"):
        for _ in range(4):
            idx = tuple(rng.integers(0, s) for s in inp[name].shape)
            plus = {k: v.copy() for k, v in inp.items()}
            minus = {k: v.copy() for k, v in inp.items()}
            plus[name][idx] += eps
            minus[name][idx] -= eps
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            assert abs(fd - g["d" + name][idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx)


def test_zero_weights_closed_form():
    """Wq = Wk = Wv = 0: every query/key/value row is its bias, attention returns the value
    bias, so Y[r] = Wo bv + bo for every row; dX = 0 and dbv = sum_r (dY Wo)."""
    b, t, e, h, d = 2, 7, 6, 2, 3
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=5)
    for k in ("wq", "wk", "wv"):
        inp[k] = np.zeros_like(inp[k])
    f, g = run_oracle(inp, h, d, False)
    want = inp["wo"].astype(np.float64) @ inp["bv"].astype(np.float64) + inp["bo"]
    np.testing.assert_allclose(f["y"], np.broadcast_to(want, f["y"].shape), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(g["dx"], 0.0, atol=1e-12)
    dyr = inp["dy"].astype(np.float64).reshape(-1, e)
    np.testing.assert_allclose(g["dbv"], (dyr @ inp["wo"].astype(np.float64)).sum(axis=0), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(g["dbq"], 0.0, atol=1e-12)  # scores are constant along each row


def test_head_layout_roundtrip():
    a = np.arange(2 * 3 * 4 * 5, dtype=np.float64).reshape(2, 3, 4, 5)
    m = lay.to_rows(a)
    assert m.shape == (8, 15)
    assert m[1 * 4 + 2, 1 * 5 + 3] == a[1, 1, 2, 3]
    np.testing.assert_array_equal(lay.from_rows(m, 2, 3, 4, 5), a)


@pytest.mark.parametrize("kind", ["bias_first_row_per_tile", "transposed_weight", "wrong_head_layout",
                                  "missing_value_path_in_dx"])
def test_planted_layer_mistakes_are_caught(kind):
    """Mistakes planted in a copy of the oracle must fail the torch comparison."""
    b, t, e, h, d = 2, 40, 12, 2, 4  # 80 rows: more than one 32-row tile; E != H*d
    inp = lay.make_layer_inputs(b, t, e, h, d, seed=9)
    f, g = run_oracle(inp, h, d, False)
    y_ref, g_ref = torch_layer(inp, h, d, False)
    if kind == "bias_first_row_per_tile":
        # The reference's projBackwardWB bias sum (attention_proj_kernels.cu:188,194-196).
        dyr = inp["dy"].astype(np.float64).reshape(-1, e)
        bad = dyr[::32].sum(axis=0)
        assert not np.allclose(bad, g_ref["dbo"], atol=1e-6)
        np.testing.assert_allclose(g["dbo"], g_ref["dbo"], rtol=1e-9, atol=1e-10)
    elif kind == "transposed_weight":
        # W taken as [E, H*d] (the getter's label) instead of [H*d, E]: cannot even be applied
        # with E != H*d, and with a square reinterpretation it is a different product.
        x = inp["x"].astype(np.float64).reshape(-1, e)
        with pytest.raises(ValueError):
            _ = x @ inp["wq"].astype(np.float64)  # [rows, E] @ [H*d, E]: shape error
    elif kind == "wrong_head_layout":
        # Reading [B, T, H, d] as [B, H, T, d]: wrong attention rows.
        q = f["q"].transpose(0, 2, 1, 3).reshape(f["q"].shape)
        from oracle import attention_fp64 as attn
        o_bad, _ = attn.attention_fwd(q, f["k"], f["v"], False)
        y_bad = lay.to_rows(o_bad) @ inp["wo"].astype(np.float64).T + inp["bo"]
        assert not np.allclose(y_bad.reshape(y_ref.shape), y_ref, atol=1e-6)
    elif kind == "missing_value_path_in_dx":
        dx_bad = g["dx"] - (lay.to_rows(g["dv"]) @ inp["wv"].astype(np.float64)).reshape(g["dx"].shape)
        assert not np.allclose(dx_bad, g_ref["dx"], atol=1e-6)
        np.testing.assert_allclose(g["dx"], g_ref["dx"], rtol=1e-9, atol=1e-10)
