"""Pins the CPU oracle before anything is checked against it (CPU only).

The oracle (``oracle/attention_fp64.py``, ``oracle/attn_online.c``) restates the math of
``flash_attention.cu``; these tests tie it to things it did not write itself:

* torch's ``scaled_dot_product_attention`` in fp64 with autograd -- the comparator of the
  reference's own test (``test_flash_attention.py:49``);
* the C online-softmax restatement (tile loop as in ``flash_attention.cu:97-161``);
* closed forms and invariants of attention;
* central finite differences of ``sum(O * dO)``;
* a planted-mistake check: plausible bugs put into a copy of the oracle make at
  least one of the checks fail, so the checks have teeth.
"""
import numpy as np
import pytest
import torch

from oracle import attention_fp64 as ora
from oracle import c_oracle, torch_cpu

SHAPES = [(1, 2, 17, 8), (2, 3, 64, 32), (1, 1, 40, 16), (1, 2, 1, 8), (1, 1, 33, 64)]


def _inputs(shape, seed=0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(shape) for _ in range(4)]


def _maxdiff(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b)))) if np.size(a) else 0.0


@pytest.fixture(scope="module", autouse=True)
def _c_oracle_built():
    import subprocess
    import os

    subprocess.run(["make", "-s", "-C", os.path.dirname(c_oracle.__file__)], check=True)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_dense_oracle_matches_torch_sdpa_fp64(shape, causal):
    q, k, v, do = _inputs(shape, seed=hash((shape, causal)) % 1000)
    got = ora.attention_fwd_bwd(q, k, v, do, causal)
    ref = torch_cpu.fwd_bwd(q, k, v, do, causal)
    for name in ("o", "lse", "dq", "dk", "dv"):
        assert _maxdiff(got[name], ref[name]) < 1e-10, name


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("tile", [32, 7])
def test_c_online_oracle_matches_dense(shape, causal, tile):
    q, k, v, do = _inputs(shape, seed=7)
    o, lse = c_oracle.fwd(q, k, v, causal, tile=tile)
    dq, dk, dv = c_oracle.bwd(q, k, v, o, do, lse, causal)
    ref = ora.attention_fwd_bwd(q, k, v, do, causal)
    for name, val in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert _maxdiff(val, ref[name]) < 1e-11, name


# ----------------------------------------------------------------------------------
# closed forms and invariants
# ----------------------------------------------------------------------------------

def test_single_token():
    q, k, v, do = _inputs((2, 3, 1, 16), seed=1)
    for causal in (False, True):
        r = ora.attention_fwd_bwd(q, k, v, do, causal)
        assert _maxdiff(r["o"], v) < 1e-14
        assert _maxdiff(r["dv"], do) < 1e-14
        assert np.max(np.abs(r["dq"])) < 1e-14 and np.max(np.abs(r["dk"])) < 1e-14
        s00 = np.sum(q * k, axis=-1) / 4.0
        assert _maxdiff(r["lse"], s00) < 1e-13


def test_causal_first_row_is_v0():
    q, k, v, do = _inputs((1, 2, 24, 8), seed=2)
    o, lse = ora.attention_fwd(q, k, v, causal=True)
    assert _maxdiff(o[:, :, 0], v[:, :, 0]) < 1e-14
    assert _maxdiff(lse[:, :, 0], np.sum(q[:, :, 0] * k[:, :, 0], -1) / np.sqrt(8)) < 1e-13


@pytest.mark.parametrize("causal", [False, True])
def test_equal_keys_give_mean_of_values_and_zero_dq(causal):
    q, k, v, do = _inputs((1, 2, 20, 8), seed=3)
    k[:] = k[:, :, :1]
    r = ora.attention_fwd_bwd(q, k, v, do, causal)
    t = q.shape[2]
    if causal:
        mean = np.cumsum(v, axis=2) / np.arange(1, t + 1)[None, None, :, None]
    else:
        mean = np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape)
    assert _maxdiff(r["o"], mean) < 1e-13
    assert np.max(np.abs(r["dq"])) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_constant_values(causal):
    q, k, v, do = _inputs((1, 2, 20, 8), seed=4)
    c = np.linspace(-1, 1, 8)
    v[:] = c
    r = ora.attention_fwd_bwd(q, k, v, do, causal)
    assert _maxdiff(r["o"], np.broadcast_to(c, v.shape)) < 1e-13
    assert np.max(np.abs(r["dq"])) < 1e-12 and np.max(np.abs(r["dk"])) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_key_shift_invariance(causal):
    q, k, v, _ = _inputs((1, 2, 20, 8), seed=5)
    o1, _ = ora.attention_fwd(q, k, v, causal)
    o2, _ = ora.attention_fwd(q, k + np.linspace(0.5, 2.0, 8), v, causal)
    assert _maxdiff(o1, o2) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_gradient_sums(causal):
    q, k, v, do = _inputs((2, 2, 30, 8), seed=6)
    r = ora.attention_fwd_bwd(q, k, v, do, causal)
    assert np.max(np.abs(r["dk"].sum(axis=2))) < 1e-12
    assert _maxdiff(r["dv"].sum(axis=2), do.sum(axis=2)) < 1e-12


def test_noncausal_permutation_invariance():
    q, k, v, _ = _inputs((1, 2, 20, 8), seed=8)
    perm = np.random.default_rng(0).permutation(20)
    o1, l1 = ora.attention_fwd(q, k, v, False)
    o2, l2 = ora.attention_fwd(q, k[:, :, perm], v[:, :, perm], False)
    assert _maxdiff(o1, o2) < 1e-13 and _maxdiff(l1, l2) < 1e-13


@pytest.mark.parametrize("causal", [False, True])
def test_zero_queries_give_log_count(causal):
    _, k, v, _ = _inputs((1, 1, 12, 4), seed=9)
    q = np.zeros_like(k)
    o, lse = ora.attention_fwd(q, k, v, causal)
    n = np.arange(1, 13) if causal else np.full(12, 12)
    assert _maxdiff(lse[0, 0], np.log(n)) < 1e-14


@pytest.mark.parametrize("causal", [False, True])
def test_finite_differences(causal):
    q, k, v, do = _inputs((1, 1, 5, 3), seed=10)
    r = ora.attention_fwd_bwd(q, k, v, do, causal)

    def loss(qq, kk, vv):
        o, _ = ora.attention_fwd(qq, kk, vv, causal)
        return float(np.sum(o * do))

    h = 1e-6
    for name, arr in (("dq", q), ("dk", k), ("dv", v)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a_p, a_m = arr.copy(), arr.copy()
            a_p[idx] += h
            a_m[idx] -= h
            args_p = [q, k, v]
            args_m = [q, k, v]
            pos = {"dq": 0, "dk": 1, "dv": 2}[name]
            args_p[pos], args_m[pos] = a_p, a_m
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        assert _maxdiff(num, r[name]) < 1e-7, name


def test_round_to_bf16_matches_torch():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32),
                        np.array([1.0, 1.00390625, 1.01171875, -2.5, 0.0, 3.0e-39], np.float32)])
    # values exactly halfway between two bf16 numbers (ties to even)
    ties = (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    ref = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ora.round_to_bf16(x), ref)


def test_round_to_f16_matches_torch():
    rng = np.random.default_rng(12)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 8,
                        np.array([1.0, 1.00048828125, 65504.0, 6.0e-8, -0.0, 1e-3], np.float32)])
    # values exactly halfway between two binary16 numbers in [1, 2) (ties to even)
    ties = (np.float32(1.0) + (np.arange(0, 200, dtype=np.float32) * 2 + 1) * np.float32(2.0 ** -11))
    x = np.concatenate([x, ties, -ties])
    ref = torch.tensor(x).to(torch.float16).to(torch.float32).numpy()
    assert np.array_equal(ora.round_to_f16(x), ref)


# ----------------------------------------------------------------------------------
# planted mistakes: each plausible bug must trip a check above
# ----------------------------------------------------------------------------------

def _mutant_bwd(kind):
    def bwd(q, k, v, o, do, lse, causal=False):
        d = q.shape[-1]
        s = ora.scores(q, k, causal)
        p = np.exp(s - lse[..., None])
        dv = np.swapaxes(p, -1, -2) @ do
        dp = do @ np.swapaxes(v, -1, -2)
        delta = np.sum(do * o, axis=-1)
        if kind == "drop_delta":
            ds = p * dp
        else:
            ds = p * (dp - delta[..., None])
        dq = ds @ k / np.sqrt(d)
        if kind == "reference_dk":
            # flash_attention.cu:312-313: row sum of dS times Q of the same row, added to key row
            dk = np.sum(ds, axis=-1, keepdims=True) * q / np.sqrt(d)
        elif kind == "scale_mul":
            dk = np.swapaxes(ds, -1, -2) @ q * np.sqrt(d)
        else:
            dk = np.swapaxes(ds, -1, -2) @ q / np.sqrt(d)
        return dq, dk, dv
    return bwd


def _mutant_fwd(kind):
    def fwd(q, k, v, causal=False):
        d = q.shape[-1]
        if kind == "transposed_mask":
            s = q @ np.swapaxes(k, -1, -2) / np.sqrt(d)
            t = s.shape[-1]
            if causal:
                s = np.where(np.tril(np.ones((t, t), bool), k=-1), -np.inf, s)
        elif kind == "scale_mul":
            s = q @ np.swapaxes(k, -1, -2) * np.sqrt(d)
        else:
            s = ora.scores(q, k, causal)
        m = s.max(-1)
        p = np.exp(s - m[..., None])
        l = p.sum(-1)
        return (p @ v) / l[..., None], m + np.log(l)
    return fwd


@pytest.mark.parametrize("kind", ["drop_delta", "reference_dk", "scale_mul"])
def test_planted_backward_mistakes_are_caught(kind):
    q, k, v, do = _inputs((1, 2, 17, 8), seed=12)
    o, lse = ora.attention_fwd(q, k, v, True)
    dq, dk, dv = _mutant_bwd(kind)(q, k, v, o, do, lse, True)
    ref = torch_cpu.fwd_bwd(q, k, v, do, True)
    worst = max(_maxdiff(dq, ref["dq"]), _maxdiff(dk, ref["dk"]), _maxdiff(dv, ref["dv"]))
    assert worst > 1e-3, f"mutant {kind} not detected by the torch comparison"
    sums_ok = np.max(np.abs(dk.sum(axis=2))) < 1e-12
    if kind == "drop_delta":
        assert not sums_ok, f"mutant {kind} not detected by the sum(dK)=0 invariant"
    if kind == "reference_dk":
        # the defective dK is identically zero (rows of dS sum to zero), so the sum
        # invariant cannot see it; the equal-keys closed form (dQ = 0) does not involve
        # dK either -- only the library comparison above pins dK against this bug.
        assert np.max(np.abs(dk)) < 1e-12


@pytest.mark.parametrize("kind", ["transposed_mask", "scale_mul"])
def test_planted_forward_mistakes_are_caught(kind):
    q, k, v, do = _inputs((1, 2, 17, 8), seed=13)
    o, lse = _mutant_fwd(kind)(q, k, v, True)
    ref = torch_cpu.fwd_bwd(q, k, v, do, True)
    assert max(_maxdiff(o, ref["o"]), _maxdiff(lse, ref["lse"])) > 1e-3
    if kind == "transposed_mask":
        # the causal first-row closed form catches it independently of torch
        assert _maxdiff(o[:, :, 0], v[:, :, 0]) > 1e-3
