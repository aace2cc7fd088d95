"""Tensor methods of the host module (casts, broadcasting arithmetic and comparisons, unary
minus, reductions, transpose, kron, matmul) on every tensor class, against numpy.

numpy is the oracle: integer and bool results and casts are compared bit for bit; floating
arithmetic within the storage type's rounding of the result (fp32 1e-6, bf16 8e-3, fp16 1e-3
relative to the largest value, fp64 1e-13), and matrix products within their K-term
accumulation (fp32 2e-5, bf16 2e-2, fp16 4e-3, fp64 1e-12).  bf16 values are rounded by the
oracle's round_to_bf16; fp64 -> bf16 casts by an exact 8-significant-bit rounding below.
"""
import numpy as np
import pytest

import cudatransformer_amd  # noqa: F401  (torch first, then the native libraries)
from cudatransformer_amd import cuda_transformer as ctm
from oracle import attention_fp64 as ora

FLOAT = ["Float", "Double", "Half", "BFloat"]
INT = ["Int", "Long", "Short", "Byte"]
NP_INT = {"Int": np.int32, "Long": np.int64, "Short": np.int16, "Byte": np.int8}
ROUND = {"Float": lambda a: np.asarray(a, np.float32).astype(np.float64),
         "Double": lambda a: np.asarray(a, np.float64),
         "Half": lambda a: ora.round_to_f16(a).astype(np.float64),
         "BFloat": lambda a: ora.round_to_bf16(a).astype(np.float64)}
REL = {"Float": 1e-6, "Double": 1e-13, "Half": 1e-3, "BFloat": 8e-3}
MM_REL = {"Float": 2e-5, "Double": 1e-12, "Half": 4e-3, "BFloat": 2e-2}


def say(msg):
    print(msg, flush=True)


def tensor(kind, a):
    return getattr(ctm, f"{kind}Tensor").fromNumpy(a)


def close(got, want, rel, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    scale = max(float(np.max(np.abs(want))), 1e-30) if want.size else 1.0
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    assert err <= rel * scale, f"{what}: err {err:.3e} scale {scale:.3e}"


def bf16_from_f64(x):
    """fp64 -> bf16 correctly rounded (8 significant bits, ties to even; normal range)."""
    m, e = np.frexp(np.asarray(x, np.float64))
    return np.ldexp(np.round(m * 256.0), e - 8)


def test_tensor_classes_and_methods_exist():
    for kind in FLOAT + INT + ["Bool"]:
        cls = getattr(ctm, f"{kind}Tensor")
        for meth in ("float", "half", "bfloat", "double", "int", "long", "short", "byte", "bool", "sum", "mean",
                     "max", "min", "manhattan", "norm", "norm_l1", "norm_l2", "transpose", "kron", "matmul",
                     "reduce", "cpu", "__add__", "__radd__", "__sub__", "__rsub__", "__mul__", "__rmul__",
                     "__truediv__", "__rtruediv__", "__mod__", "__matmul__", "__rmatmul__", "__neg__", "__eq__",
                     "__lt__", "__ge__"):
            assert hasattr(cls, meth), (kind, meth)
    assert {m for m in dir(ctm.ReductionOp) if m.isupper()} >= {"SUM", "MEAN", "MAX", "MIN", "NORM_L1", "NORM_L2"}


@pytest.mark.gpu
def test_integer_and_bool_tensors_round_trip():
    rng = np.random.default_rng(1)
    for kind, npt in NP_INT.items():
        info = np.iinfo(npt)
        a = rng.integers(info.min, info.max, size=(3, 7), dtype=npt, endpoint=True)
        t = tensor(kind, a)
        back = t.numpy()
        assert back.dtype == npt and np.array_equal(back, a)
        assert t.clone().cpu() == a.ravel().tolist()
        assert getattr(ctm, f"{kind}Tensor").fromNumpy(a[:1, :1].copy()).item() == int(a[0, 0])
    b = rng.integers(0, 2, size=(5, 4)).astype(bool)
    tb = ctm.BoolTensor.fromNumpy(b)
    assert tb.numpy().dtype == np.bool_ and np.array_equal(tb.numpy(), b)
    assert ctm.BoolTensor.fromNumpy(np.array([True])).item() is True
    z = ctm.LongTensor([2, 3])
    z.fill(2 ** 40 + 3)
    assert np.all(z.numpy() == 2 ** 40 + 3)


@pytest.mark.gpu
@pytest.mark.parametrize("src", FLOAT + INT + ["Bool"])
def test_casts(src):
    say(f"casts from {src}")
    rng = np.random.default_rng(2)
    if src in FLOAT:
        a = ROUND[src](np.concatenate([rng.standard_normal(500) * 50, [0.0, -0.0, 1.5, -2.5, 127.9, -128.7, 1e-3]]))
        a = a.astype(np.float64 if src == "Double" else np.float32)
    elif src == "Bool":
        a = rng.integers(0, 2, 300).astype(bool)
    else:
        info = np.iinfo(NP_INT[src])
        a = rng.integers(max(info.min, -30000), min(info.max, 30000), 500, dtype=NP_INT[src], endpoint=True)
    t = tensor(src, a)
    x = a.astype(np.float64)
    close(t.double().numpy(), x, 0.0, "double")
    assert np.array_equal(t.float().numpy(), x.astype(np.float32))
    assert np.array_equal(t.half().numpy(), ora.round_to_f16(x) if src != "Double" else x.astype(np.float16).astype(np.float32))
    bf = t.bfloat().numpy().astype(np.float64)
    assert np.array_equal(bf, bf16_from_f64(x)), "bfloat"
    assert np.array_equal(t.bool().numpy(), x != 0)
    for kind, npt in NP_INT.items():
        got = getattr(t, {"Int": "int", "Long": "long", "Short": "short", "Byte": "byte"}[kind])().numpy()
        want = np.trunc(x).astype(np.int64).astype(npt)  # truncation toward zero, wrap-around
        assert got.dtype == npt and np.array_equal(got, want), kind


@pytest.mark.gpu
def test_f64_to_narrow_casts_round_once():
    """Values just above a bf16 / fp16 rounding tie: rounding through fp32 would land on the
    tie and round to even (down); the direct conversion rounds up."""
    k = np.arange(1, 60, dtype=np.float64)
    bf_ties = 1.0 + (2 * k + 1) * 2.0 ** -8  # halfway between bf16 neighbours in [1, 2)
    f16_ties = 1.0 + (2 * k + 1) * 2.0 ** -11
    x = np.concatenate([bf_ties + 2.0 ** -40, f16_ties + 2.0 ** -40, bf_ties, -bf_ties - 2.0 ** -40])
    t = ctm.DoubleTensor.fromNumpy(x)
    assert np.array_equal(t.bfloat().numpy().astype(np.float64), bf16_from_f64(x))
    assert np.array_equal(t.half().numpy(), x.astype(np.float16).astype(np.float32))


SHAPE_PAIRS = [((4, 5), (4, 5)), ((3, 1, 5), (4, 1)), ((6,), (2, 3, 6)), ((2, 1, 3, 1), (1, 4, 1, 5)), ((0, 3), (3,))]


@pytest.mark.gpu
@pytest.mark.parametrize("kind", FLOAT + INT + ["Bool"])
def test_broadcast_arithmetic_and_comparisons(kind):
    say(f"binary {kind}")
    rng = np.random.default_rng(3)
    for sa, sb in SHAPE_PAIRS:
        if kind in FLOAT:
            a, b = ROUND[kind](rng.standard_normal(sa) * 3), ROUND[kind](rng.standard_normal(sb) * 3 + 0.5)
            b[b == 0] = 1.0
        elif kind == "Bool":
            a, b = rng.integers(0, 2, sa).astype(bool), rng.integers(0, 2, sb).astype(bool)
        else:
            a = rng.integers(-100, 100, sa).astype(NP_INT[kind])
            b = rng.integers(-9, 9, sb).astype(NP_INT[kind])
        ta, tb = tensor(kind, a.astype(np.float32) if kind in ("Half", "BFloat") else a), \
            tensor(kind, b.astype(np.float32) if kind in ("Half", "BFloat") else b)
        x, y = a.astype(np.float64), b.astype(np.float64)
        for name, fn in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", None), ("mod", None)):
            got = {"add": ta + tb, "sub": ta - tb, "mul": ta * tb, "div": ta / tb, "mod": ta % tb}[name].numpy()
            if kind in FLOAT:
                want = np.zeros(np.broadcast_shapes(sa, sb)) if name == "mod" else (
                    x / y if name == "div" else fn(x, y))
                close(got, ROUND[kind](want), REL[kind], f"{kind} {name} {sa} {sb}")
            else:
                xi, yi = np.broadcast_arrays(x.astype(np.int64), y.astype(np.int64))
                safe = np.where(yi == 0, 1, yi)
                want = {"add": xi + yi, "sub": xi - yi, "mul": xi * yi,
                        "div": np.where(yi == 0, 0, np.trunc(xi / safe).astype(np.int64)),
                        "mod": np.where(yi == 0, 0, np.fmod(xi, safe))}[name]
                if kind == "Bool":
                    assert np.array_equal(got, want != 0), (name, sa, sb)
                else:
                    assert np.array_equal(got, want.astype(NP_INT[kind])), (kind, name, sa, sb)
        for name, fn in (("eq", np.equal), ("ne", np.not_equal), ("lt", np.less), ("le", np.less_equal),
                         ("gt", np.greater), ("ge", np.greater_equal)):
            got = {"eq": ta == tb, "ne": ta != tb, "lt": ta < tb, "le": ta <= tb, "gt": ta > tb,
                   "ge": ta >= tb}[name]
            assert isinstance(got, ctm.BoolTensor)
            assert np.array_equal(got.numpy(), fn(x, y)), (kind, name, sa, sb)
    with pytest.raises(ValueError):
        tensor(kind, np.zeros((2, 3), np.float32 if kind in FLOAT else (bool if kind == "Bool" else NP_INT[kind]))) + \
            tensor(kind, np.zeros((4,), np.float32 if kind in FLOAT else (bool if kind == "Bool" else NP_INT[kind])))


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["Float", "Double", "Int", "Half"])
def test_scalar_operators(kind):
    rng = np.random.default_rng(4)
    a = rng.integers(1, 50, (4, 6)).astype(np.float64) * (1 if kind != "Float" else 0.5)
    t = tensor(kind, a.astype(np.int32) if kind == "Int" else a)
    x = a.astype(np.int64) if kind == "Int" else a
    checks = {"t+3": (t + 3, x + 3), "3+t": (3 + t, x + 3), "t-2": (t - 2, x - 2), "10-t": (10 - t, 10 - x),
              "t*4": (t * 4, x * 4), "4*t": (4 * t, x * 4), "-t": (-t, -x)}
    if kind == "Int":
        checks.update({"t/3": (t / 3, x // 3), "100/t": (100 / t, 100 // x), "t%7": (t % 7, x % 7),
                       "t+2.9": (t + 2.9, x + 2)})  # the scalar becomes the storage type first
    else:
        checks.update({"t/4": (t / 4, x / 4), "2/t": (2 / t, 2 / x)})
    for what, (got, want) in checks.items():
        got = got.numpy().astype(np.float64)
        if kind in ("Int",):
            assert np.array_equal(got, want), what
        else:
            close(got, ROUND[kind](want), REL[kind], what)
    assert np.array_equal((t > 20).numpy(), x > 20) and np.array_equal((t == 7).numpy(), x == 7)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", FLOAT + ["Int", "Long", "Bool"])
def test_reductions(kind):
    say(f"reductions {kind}")
    rng = np.random.default_rng(5)
    shape = (3, 4, 130)
    if kind in FLOAT:
        a = ROUND[kind](rng.standard_normal(shape))
    elif kind == "Bool":
        a = rng.integers(0, 2, shape).astype(bool)
    else:
        a = rng.integers(-1000, 1000, shape).astype(NP_INT[kind])
    t = tensor(kind, a.astype(np.float32) if kind in ("Half", "BFloat") else a)
    x = a.astype(np.float64)
    fns = {"sum": np.sum, "mean": np.mean, "max": np.max, "min": np.min,
           "norm_l1": lambda v, axis=None: np.sum(np.abs(v), axis=axis),
           "manhattan": lambda v, axis=None: np.sum(np.abs(v), axis=axis),
           "norm_l2": lambda v, axis=None: np.sqrt(np.sum(v * v, axis=axis)),
           "norm": lambda v, axis=None: np.sqrt(np.sum(v * v, axis=axis))}
    if kind == "Bool":
        del fns["mean"]  # a bool mean is integer division of the count: not numpy's any()
    for name, fn in fns.items():
        for dim in (-1, 0, 1, 2):
            got = getattr(t, name)(dim).numpy().astype(np.float64)
            want = np.atleast_1d(fn(x) if dim < 0 else fn(x, axis=dim))
            if kind == "Bool":
                want = want != 0
                assert np.array_equal(got, want), (name, dim)
            elif kind in ("Int", "Long"):
                want = np.trunc(want) if name in ("mean", "norm_l2", "norm") else want
                assert np.array_equal(got, want.astype(np.int64).astype(NP_INT[kind])), (name, dim)
            else:
                close(got, ROUND[kind](want), max(REL[kind], 1e-6 if kind != "Double" else 1e-13), f"{name} {dim}")
    got = t.reduce([0, 2], ctm.ReductionOp.SUM).numpy().astype(np.float64)
    want = x.sum(axis=(0, 2))
    if kind in FLOAT:
        close(got, ROUND[kind](want), max(REL[kind], 1e-6), "reduce [0, 2]")
    elif kind != "Bool":
        assert np.array_equal(got, want)


@pytest.mark.gpu
def test_large_reductions_are_deterministic():
    x = np.random.default_rng(6).standard_normal((3_000_000,)).astype(np.float32)
    t = ctm.FloatTensor.fromNumpy(x)
    s1, s2 = t.sum().item(), t.sum().item()
    assert s1 == s2
    assert abs(s1 - x.astype(np.float64).sum()) <= 1e-6 * np.abs(x).sum()
    m = ctm.FloatTensor.fromNumpy(x.reshape(1000, 3000))
    close(m.sum(0).numpy(), x.reshape(1000, 3000).astype(np.float64).sum(0), 1e-5, "column sums")
    close(m.max(1).numpy(), x.reshape(1000, 3000).max(1), 0.0, "row max")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["Float", "Half", "Long", "Byte", "Bool"])
def test_transpose_and_kron(kind):
    rng = np.random.default_rng(7)
    npt = {"Float": np.float32, "Half": np.float32, "Long": np.int64, "Byte": np.int8, "Bool": bool}[kind]
    a = (rng.integers(-5, 5, (2, 3, 4, 5)) if kind != "Bool" else rng.integers(0, 2, (2, 3, 4, 5))).astype(npt)
    t = tensor(kind, a)
    for perm in ([3, 1, 0, 2], [0, 1, 2, 3], [1, 0, 3, 2]):
        assert np.array_equal(t.transpose(perm).numpy(), a.transpose(perm)), perm
    assert np.array_equal(t.transpose(1, 3).numpy(), np.swapaxes(a, 1, 3))
    # the last two axes swapped: the tiled transpose kernel (ragged tile edges included)
    for shape in ((3, 70, 130), (1000, 7), (2, 1, 64, 65)):
        c = (rng.integers(-5, 5, shape) if kind != "Bool" else rng.integers(0, 2, shape)).astype(npt)
        tc = tensor(kind, c)
        assert np.array_equal(tc.transpose(len(shape) - 2, len(shape) - 1).numpy(), np.swapaxes(c, -1, -2)), shape
    with pytest.raises(ValueError):
        t.transpose([0, 0, 1, 2])
    b = (rng.integers(-3, 3, (2, 1, 3, 2)) if kind != "Bool" else rng.integers(0, 2, (2, 1, 3, 2))).astype(npt)
    want = np.kron(a.astype(np.int64), b.astype(np.int64))
    got = t.kron(tensor(kind, b)).numpy()
    assert np.array_equal(got.astype(np.int64), want if kind != "Bool" else (want != 0)), kind


@pytest.mark.gpu
@pytest.mark.parametrize("kind", FLOAT + ["Int", "Long"])
@pytest.mark.parametrize("shapes", [((5, 7), (7, 3)), ((4, 33, 20), (4, 20, 12)), ((4, 33, 32), (4, 32, 12)),
                                    ((3, 2, 16, 64), (64, 32)),
                                    ((8, 128), (128, 256)), ((2, 3, 0), (0, 4))])
def test_matmul(kind, shapes):
    sa, sb = shapes
    say(f"matmul {kind} {sa} {sb}")
    rng = np.random.default_rng(8)
    if kind in FLOAT:
        a, b = ROUND[kind](rng.standard_normal(sa)), ROUND[kind](rng.standard_normal(sb))
        ta, tb = tensor(kind, a if kind == "Double" else a.astype(np.float32)), \
            tensor(kind, b if kind == "Double" else b.astype(np.float32))
    else:
        a, b = rng.integers(-50, 50, sa).astype(NP_INT[kind]), rng.integers(-50, 50, sb).astype(NP_INT[kind])
        ta, tb = tensor(kind, a), tensor(kind, b)
    got = (ta @ tb).numpy()
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert got.shape == want.shape
    if kind in FLOAT:
        close(got, want, MM_REL[kind], f"{kind} {sa}@{sb}")
    else:
        assert np.array_equal(got, want.astype(np.int64).astype(NP_INT[kind]))
    assert np.array_equal(ta.matmul(tb).numpy(), got)
    with pytest.raises(ValueError):
        ta @ tensor(kind, np.zeros((3, 5), np.float32 if kind in ("Float", "Half", "BFloat") else
                                   (np.float64 if kind == "Double" else NP_INT[kind])))
