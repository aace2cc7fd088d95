"""GPU parity of the ctattn kernels against the fp64 oracle, through the C-ABI.

Tolerances (fixed by the build's target): fp32 max|x - g| <= 1e-4 on each of O, LSE, dQ,
dK, dV; bf16 max|x - g| / max|g| <= 2e-2 per tensor, g computed from the bf16-rounded
inputs.  Every kernel policy is exercised: POLICY_AUTO (MFMA where supported, dQ by fp32
atomics), POLICY_DETERMINISTIC (MFMA, ordered dQ reduction) and POLICY_GENERIC.
"""
import glob
import os
import sys

import numpy as np
import pytest
import torch

import cudatransformer_amd as ct
from oracle import attention_fp64 as ora

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
F32_TOL = 1e-4
BF16_REL_TOL = 2e-2
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(params=[ct.POLICY_AUTO, ct.POLICY_GENERIC, ct.POLICY_DETERMINISTIC],
                ids=["auto", "generic", "deterministic"])
def policy(request):
    prev = ct.set_policy(request.param)
    yield request.param
    ct.set_policy(prev)


def run_gpu(q, k, v, do, causal, dtype, fastest=False):
    """Forward + backward on the GPU; fastest: the backward gets the workspace of its fastest
    path (ctattn_bwd_workspace_bytes_max), else the default one."""
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(td)
                       for a in (q, k, v, do))
    o, lse = ct.flash_attn_fwd(tq, tk, tv, causal)
    b, h, t, d = tq.shape
    ws = torch.empty(ct._capi.bwd_workspace_bytes(td, b, h, t, d, causal, fastest=fastest), dtype=torch.uint8,
                     device=DEV)
    dq, dk, dv = ct.flash_attn_bwd(tq, tk, tv, o, tdo, lse, causal, workspace=ws)
    torch.cuda.synchronize()
    f = lambda t: t.float().cpu().numpy().astype(np.float64)  # noqa: E731
    return {"o": f(o), "lse": f(lse), "dq": f(dq), "dk": f(dk), "dv": f(dv)}


def assert_close(got, want, dtype, ctx):
    # dQ and dK vanish in exact arithmetic where a row sees one key (T = 1: dS = P (dP - delta)
    # = 0); their bf16 scale then falls back to 1e-4 of the dV scale instead of the fp64 zero.
    floor = {"dq": 1e-4, "dk": 1e-4}
    dv_scale = float(np.max(np.abs(want["dv"]))) if want["dv"].size else 0.0
    for key in ("o", "lse", "dq", "dk", "dv"):
        g, w = got[key], want[key]
        assert g.shape == w.shape, (ctx, key)
        assert np.all(np.isfinite(g)), f"{ctx} {key}: non-finite values"
        err = float(np.max(np.abs(g - w))) if g.size else 0.0
        if dtype == "f32":
            assert err <= F32_TOL, f"{ctx} {key}: max abs err {err:.3e} > {F32_TOL}"
        else:
            scale = max(float(np.max(np.abs(w))) if w.size else 0.0, floor.get(key, 0.0) * dv_scale, 1e-30)
            rel = err / scale
            assert rel <= BF16_REL_TOL, f"{ctx} {key}: rel err {rel:.3e} > {BF16_REL_TOL}"


@pytest.mark.parametrize("path", GOLDEN, ids=os.path.basename)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_golden_fixture(path, causal, policy):
    z = np.load(path)
    dtype = "bf16" if path.endswith("_bf16.npz") else "f32"
    tag = "causal" if causal else "full"
    say(f"golden {os.path.basename(path)} causal={causal} policy={policy}")
    got = run_gpu(z["q"], z["k"], z["v"], z["do"], causal, dtype)
    want = {key: z[f"{key}_{tag}"].astype(np.float64) for key in ("o", "lse", "dq", "dk", "dv")}
    assert_close(got, want, dtype, os.path.basename(path))


SHAPES = [
    (2, 3, 1, 64),
    (1, 2, 33, 32),
    (2, 3, 257, 64),
    (1, 2, 300, 128),
    (1, 1, 65, 48),
    (1, 1, 70, 256),
    (1, 2, 129, 8),
    (2, 2, 300, 32),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_parity_vs_oracle(shape, causal, dtype, policy):
    seed = 100 + SHAPES.index(shape)
    std = 1.0 if dtype == "f32" else 0.5
    q, k, v, do = ora.make_inputs(shape, seed, std=std, dtype=dtype)
    say(f"parity shape={shape} causal={causal} dtype={dtype} policy={policy}")
    got = run_gpu(q, k, v, do, causal, dtype)
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    assert_close(got, want, dtype, f"{shape} causal={causal}")


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_c2_c3_full_size_f32(causal):
    """Configs 2/3: B8 H12 T1024 d64 fp32, N(0,1) seed 2 -- fwd and fwd+bwd at full size."""
    shape = (8, 12, 1024, 64)
    q, k, v, do = ora.make_inputs(shape, seed=2)
    say(f"c2/c3 full size causal={causal}")
    got = run_gpu(q, k, v, do, causal, "f32")
    want = ora.attention_fwd_bwd(q, k, v, do, causal, chunk_heads=12)
    assert_close(got, want, "f32", f"c3 causal={causal}")


C4_SHAPE = (1, 32, 8192, 128)
# Eight of the 32 heads, spread over the range, checked against the oracle two per test (the
# fp64 oracle takes ~10 s per head at T = 8192); every head through the invariants.
C4_HEAD_PAIRS = [(0, 4), (9, 13), (18, 22), (27, 31)]


@pytest.fixture(scope="module")
def c4_run():
    """Config 4: B1 H32 T8192 d128 bf16, N(0, 0.5^2) seed 4, causal -- one GPU fwd+bwd shared
    by the c4 tests, with the workspace of the fastest path (the dK/dV kernel stores dS)."""
    q, k, v, do = ora.make_inputs(C4_SHAPE, seed=4, std=0.5, dtype="bf16")
    say("c4 full size bf16")
    got = run_gpu(q, k, v, do, True, "bf16", fastest=True)
    return q, k, v, do, got


@pytest.mark.parametrize("heads", C4_HEAD_PAIRS, ids=lambda h: f"h{h[0]}_{h[1]}")
def test_c4_long_context_bf16_vs_oracle(c4_run, heads):
    q, k, v, do, got = c4_run
    for h in heads:
        say(f"c4 head {h} vs oracle")
        sl = lambda a: a[:, h:h + 1]  # noqa: E731
        want = ora.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), True, chunk_heads=1)
        assert_close({kk: sl(vv) for kk, vv in got.items()}, want, "bf16", f"c4 head {h}")


def test_c4_long_context_bf16_invariants(c4_run):
    """Per (b, h): sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i.  The exact sums are 0 and
    sum_i dO_i; what remains is the bf16 rounding of dK / dV / O, measured on the fp64 oracle
    at this shape (head 0) as 0.0043 (dK rounding) + 0.0046 (delta from the rounded O) times
    sqrt(T) * rms(dK) and 0.005 sqrt(T) * rms(dV).  The bound is 0.05 sqrt(T) * rms per head;
    a backward that drops delta from dS exceeds it 55-fold (2.8 sqrt(T) * rms)."""
    q, k, v, do, got = c4_run
    t = C4_SHAPE[2]
    dk, dv = got["dk"], got["dv"]
    rms_k = np.sqrt(np.mean(dk ** 2, axis=(2, 3)))        # [B, H]
    rms_v = np.sqrt(np.mean(dv ** 2, axis=(2, 3)))
    assert np.all(rms_k > 0) and np.all(rms_v > 0)
    sum_k = np.max(np.abs(dk.sum(axis=2)), axis=-1)       # [B, H]
    do_sum = ora.cast_inputs([do], "bf16")[0].sum(axis=2)
    sum_v = np.max(np.abs(dv.sum(axis=2) - do_sum), axis=-1)
    bad_k = np.argwhere(sum_k > 0.05 * np.sqrt(t) * rms_k)
    bad_v = np.argwhere(sum_v > 0.05 * np.sqrt(t) * rms_v)
    assert bad_k.size == 0, f"sum dK != 0 at (b, h) {bad_k.tolist()}: {sum_k.max():.3e}"
    assert bad_v.size == 0, f"sum dV != sum dO at (b, h) {bad_v.tolist()}: {sum_v.max():.3e}"


@pytest.mark.parametrize("pol", [ct.POLICY_AUTO, ct.POLICY_DETERMINISTIC], ids=["auto", "deterministic"])
@pytest.mark.parametrize("shape", [(1, 2, 1100, 64), (1, 2, 1100, 32), (4, 64, 300, 64), (4, 64, 300, 32)],
                         ids=lambda s: "x".join(map(str, s)))
def test_causal_work_decompositions_f32(shape, pol):
    """Short fp32 causal grids are cut finer, long ones are not; both sides of each rule.
    Forward (d <= 64): every 128-row query block becomes two 64-row workgroups with halved
    key ranges when ceil(T / 128) * B * H <= 2 * CUs.  Backward: every key block's query rows
    are shared by two workgroups (dK / dV summed by two atomic adds each, order-independent)
    when ceil(T / bn) * B * H workgroups fit the chip at once (bn = 64 for the AUTO causal
    d >= 64 kernel, else 128; two per CU at d <= 64; the 64-key kernel with fewer than 16
    query blocks of 64 only while the grid fills at most half the chip).  The B1 H2 T1100
    shapes take the finer grids, the B4 H64 T300 ones the plain grids; both have a ragged last
    block.  Against the oracle, and dK / dV / O / LSE bitwise equal over two runs (all of them
    under DETERMINISTIC)."""
    b, h, t, d = shape
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    fwd_split = -(-t // 128) * b * h <= 2 * cus
    bn = 64 if (pol == ct.POLICY_AUTO and d >= 64) else 128
    slots = (2 if d <= 64 else 1) * cus
    blocks = -(-t // bn) * b * h
    nqb = -(-t // 64)
    bwd_split = blocks <= slots if (bn == 128 or nqb >= 16) else (nqb >= 4 and 2 * blocks <= slots)
    assert fwd_split == bwd_split == (h == 2), f"{shape} is expected on the other side of a rule ({cus} CUs)"
    q, k, v, do = ora.make_inputs(shape, seed=57)
    say(f"causal work decomposition shape={shape} policy={pol} split={fwd_split}")
    prev = ct.set_policy(pol)
    try:
        r1 = run_gpu(q, k, v, do, True, "f32")
        r2 = run_gpu(q, k, v, do, True, "f32")
    finally:
        ct.set_policy(prev)
    want = ora.attention_fwd_bwd(q, k, v, do, True, chunk_heads=16)
    assert_close(r1, want, "f32", f"{shape} split={fwd_split}")
    for key in (("o", "lse", "dk", "dv") if pol == ct.POLICY_AUTO else r1):
        assert np.array_equal(r1[key], r2[key]), key


@pytest.mark.parametrize("shape", [(16, 6, 256, 64), (4, 6, 256, 64)], ids=lambda s: "x".join(map(str, s)))
def test_short_sequence_backward_split_rule_f32(shape):
    """The fp32 64-key backward at short sequences: with fewer than 16 query blocks of 64 a key
    block is split between two workgroups only while the grid fills at most half the chip.
    B16 H6 T256 (config 5's attention: 384 key blocks) runs them whole, B4 H6 T256 (96) split.
    Against the oracle, dK / dV / O / LSE bitwise equal over two runs."""
    b, h, t, d = shape
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    split = 2 * (-(-t // 64)) * b * h <= 2 * cus
    assert split == (b == 4), f"{shape} is expected on the other side of the split rule ({cus} CUs)"
    q, k, v, do = ora.make_inputs(shape, seed=59)
    say(f"short sequence backward shape={shape} split={split}")
    r1 = run_gpu(q, k, v, do, True, "f32")
    r2 = run_gpu(q, k, v, do, True, "f32")
    want = ora.attention_fwd_bwd(q, k, v, do, True, chunk_heads=16)
    assert_close(r1, want, "f32", f"{shape} split={split}")
    for key in ("o", "lse", "dk", "dv"):
        assert np.array_equal(r1[key], r2[key]), key


@pytest.mark.parametrize("shape", [(1, 2, 1100, 128), (4, 72, 300, 128), (1, 2, 1100, 64), (4, 72, 300, 64),
                                   (1, 2, 1100, 32)], ids=lambda s: "x".join(map(str, s)))
def test_causal_forward_decompositions_bf16(shape):
    """The bf16 causal forward halves the key range of each workgroup's rows between two wave
    groups, merged through LDS, when the grid of whole workgroups fits the chip at once:
    d = 128 (256-row workgroups of two 4-wave groups alternating MFMA and softmax phases,
    one per CU) splits into 128-row workgroups when ceil(T / 256) * B * H <= CUs; d <= 64
    (128-row 4-wave workgroups, two per CU) into 64-row ones when ceil(T / 128) * B * H <=
    2 * CUs.  The B1 H2 T1100 shapes take the halved key ranges, B4 H72 T300 the whole ones;
    all have a ragged last block."""
    b, h, t, d = shape
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    split = (-(-t // 256) * b * h <= cus) if d == 128 else (-(-t // 128) * b * h <= 2 * cus)
    assert split == (h == 2), f"{shape} is expected on the other side of the split rule ({cus} CUs)"
    q, k, v, do = ora.make_inputs(shape, seed=58, std=0.5, dtype="bf16")
    say(f"bf16 causal forward decomposition shape={shape} split={split}")
    got = run_gpu(q, k, v, do, True, "bf16")
    want = ora.attention_fwd_bwd(q, k, v, do, True, chunk_heads=16)
    assert_close(got, want, "bf16", f"{shape} split={split}")


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_mfma_matches_generic(causal, d):
    shape = (2, 4, 200, d)
    q, k, v, do = ora.make_inputs(shape, seed=31)
    a = run_gpu(q, k, v, do, causal, "f32")
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        b = run_gpu(q, k, v, do, causal, "f32")
    finally:
        ct.set_policy(prev)
    for key in a:
        assert np.max(np.abs(a[key] - b[key])) <= 5e-5, key


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_deterministic_policy_is_bitwise_reproducible(dtype, causal):
    shape = (2, 3, 1000, 64)
    q, k, v, do = ora.make_inputs(shape, seed=41, dtype=dtype)
    prev = ct.set_policy(ct.POLICY_DETERMINISTIC)
    try:
        r1 = run_gpu(q, k, v, do, causal, dtype)
        r2 = run_gpu(q, k, v, do, causal, dtype)
    finally:
        ct.set_policy(prev)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_deterministic_long_sequence_f32(causal, d):
    """DETERMINISTIC fp32 beyond 8 key blocks of 128 (T > 1024): dK / dV from the 128-key
    kernel without its dQ part, dQ from the query-major kernel.  Against the oracle, and
    bitwise equal over two runs."""
    shape = (1, 2, 1100, d)
    q, k, v, do = ora.make_inputs(shape, seed=43 + d)
    say(f"deterministic long sequence shape={shape} causal={causal}")
    prev = ct.set_policy(ct.POLICY_DETERMINISTIC)
    try:
        r1 = run_gpu(q, k, v, do, causal, "f32")
        r2 = run_gpu(q, k, v, do, causal, "f32")
    finally:
        ct.set_policy(prev)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    assert_close(r1, want, "f32", f"{shape} causal={causal} deterministic")


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("shape", [(1, 3, 333, 64), (2, 2, 64, 128), (1, 2, 1100, 64), (4, 64, 300, 64),
                                   (1, 3, 333, 128)], ids=lambda s: "x".join(map(str, s)))
def test_f32_ds_path_deterministic(shape, causal):
    """fp32 DETERMINISTIC with the workspace ctattn_bwd_workspace_bytes_max asks for (d in
    {64, 128}): the 64-key kernel stores dS in the workspace and the query-major kernel
    multiplies it by K -- no atomics on dQ, no partials, no recompute.  Ragged last blocks,
    split key blocks (B1 H2 T1100) and T > 1024 included.  Against the oracle, every output
    bitwise equal over two runs, and (causal) dK / dV bitwise equal to AUTO's, whose default
    run takes the same 64-key kernel with atomic dQ."""
    q, k, v, do = ora.make_inputs(shape, seed=91)
    say(f"fp32 dS path deterministic shape={shape} causal={causal}")
    prev = ct.set_policy(ct.POLICY_DETERMINISTIC)
    try:
        r1 = run_gpu(q, k, v, do, causal, "f32", fastest=True)
        r2 = run_gpu(q, k, v, do, causal, "f32", fastest=True)
    finally:
        ct.set_policy(prev)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    assert_close(r1, want, "f32", f"{shape} causal={causal} dS path")
    if causal:
        ra = run_gpu(q, k, v, do, True, "f32")
        assert np.array_equal(ra["dk"], r1["dk"]) and np.array_equal(ra["dv"], r1["dv"])


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_f32_ds_path_auto_d128(causal):
    """AUTO takes the fp32 dS path at d = 128 on grids of at least 1024 key blocks of 64 when
    the workspace holds the tiles (B2 H64 T500: 8 x 128 key blocks, ragged): dQ then comes
    without atomics, so all five outputs are bitwise reproducible; against the oracle."""
    shape = (2, 64, 500, 128)
    q, k, v, do = ora.make_inputs(shape, seed=92)
    say(f"fp32 dS path auto shape={shape} causal={causal}")
    b, h, t, d = shape
    n = (t + 63) // 64
    ds = b * h * (n * (n + 1) // 2 if causal else n * n) * 16384
    assert ct._capi.bwd_workspace_bytes(torch.float32, b, h, t, d, causal, fastest=True) == \
        (b * h * t * 4 + 255) // 256 * 256 + ds
    r1 = run_gpu(q, k, v, do, causal, "f32", fastest=True)
    r2 = run_gpu(q, k, v, do, causal, "f32", fastest=True)
    for key in r1:
        assert np.array_equal(r1[key], r2[key]), key
    want = ora.attention_fwd_bwd(q, k, v, do, causal, chunk_heads=16)
    assert_close(r1, want, "f32", f"{shape} causal={causal} auto dS path")


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_auto_policy_reproducibility(causal):
    """AUTO: O, LSE, dK, dV bitwise reproducible; dQ (fp32 atomics across key blocks)
    reproducible up to the order of fp32 additions."""
    shape = (2, 3, 1000, 64)
    q, k, v, do = ora.make_inputs(shape, seed=42)
    r1 = run_gpu(q, k, v, do, causal, "f32")
    r2 = run_gpu(q, k, v, do, causal, "f32")
    for key in ("o", "lse", "dk", "dv"):
        assert np.array_equal(r1[key], r2[key]), key
    assert np.max(np.abs(r1["dq"] - r2["dq"])) <= 1e-5 * max(1.0, np.max(np.abs(r1["dq"])))


def test_forward_without_lse():
    lib = ct._capi.load()
    q, k, v, _ = (torch.randn(1, 2, 96, 64, device=DEV) for _ in range(4))
    o = torch.empty_like(q)
    rc = lib.ctattn_fwd(0, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), None,
                        1, 2, 96, 64, 1, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ct.last_error()
    o_ref, _ = ct.flash_attn_fwd(q, k, v, True)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)


def test_autograd_function():
    q, k, v = (torch.randn(2, 2, 64, 32, device=DEV, requires_grad=True) for _ in range(3))
    o = ct.flash_attention(q, k, v, True)
    o.sum().backward()
    qc, kc, vc = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v))
    oc = torch.nn.functional.scaled_dot_product_attention(qc, kc, vc, is_causal=True)
    oc.sum().backward()
    assert torch.max(torch.abs(o.detach().cpu().double() - oc)) < 1e-4
    for a, b in ((q, qc), (k, kc), (v, vc)):
        assert torch.max(torch.abs(a.grad.cpu().double() - b.grad)) < 1e-4


def test_invalid_inputs_raise():
    q = torch.randn(1, 2, 16, 64, device=DEV)
    with pytest.raises(ValueError):
        ct.flash_attn_fwd(q, q, q.double())
    with pytest.raises(ValueError):
        ct.flash_attn_fwd(q.transpose(1, 2), q.transpose(1, 2), q.transpose(1, 2))
    lib = ct._capi.load()
    rc = lib.ctattn_fwd(0, q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), None,
                        1, 2, 16, 300, 0, None)
    assert rc == 801


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64],
                         ids=["f32", "bf16", "f16", "f64"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_misaligned_views_take_the_generic_kernels(dtype, causal):
    """Contiguous [B, H, T, d] views one element into their storage (4, 2, 2 or 8 bytes off a
    16-byte boundary) are valid C-ABI arguments; the MFMA kernels need 16-byte-aligned
    pointers, so such calls run on the generic kernels: bitwise equal to the generic policy
    on aligned copies of the same data, and close to the oracle."""
    shape = (2, 3, 150, 64)
    say(f"misaligned views dtype={dtype} causal={causal}")
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16", torch.float64: "f64"}[dtype]
    q, k, v, do = ora.make_inputs(shape, seed=41, dtype=name)
    n = int(np.prod(shape))

    def offset_view(a):
        buf = torch.empty(n + 1, device=DEV, dtype=dtype)
        t = buf[1:].view(shape)
        t.copy_(torch.from_numpy(np.ascontiguousarray(a, np.float64)).to(DEV, dtype))
        assert t.is_contiguous() and t.data_ptr() % 16 != 0
        return t

    def run(ts):
        o, lse = ct.flash_attn_fwd(ts[0], ts[1], ts[2], causal)
        dq, dk, dv = ct.flash_attn_bwd(ts[0], ts[1], ts[2], o, ts[3], lse, causal)
        torch.cuda.synchronize()
        return {key: t.double().cpu().numpy() for key, t in
                (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))}

    got = run([offset_view(a) for a in (q, k, v, do)])
    prev = ct.set_policy(ct.POLICY_GENERIC)
    try:
        ref = run([torch.from_numpy(np.ascontiguousarray(a, np.float64)).to(DEV, dtype) for a in (q, k, v, do)])
    finally:
        ct.set_policy(prev)
    want = ora.attention_fwd_bwd(*ora.cast_inputs((q, k, v, do), name), causal)
    rel = {"f32": 1e-5, "bf16": BF16_REL_TOL, "f16": 4e-3, "f64": 1e-10}[name]
    for key in got:
        assert np.array_equal(got[key], ref[key]), key
        err = float(np.max(np.abs(got[key] - want[key])))
        assert err <= rel * max(float(np.max(np.abs(want[key]))), 1.0), (key, err)


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("shape", [(1, 3, 333, 128), (2, 2, 64, 128)], ids=lambda s: "x".join(map(str, s)))
def test_bf16_d128_ds_and_recompute_paths(shape, causal, fmt):
    """bf16 at d = 128 stores dS in the workspace and the dQ kernel multiplies it by K when the
    workspace ctattn_bwd_workspace_bytes_max asks for is given; a workspace without the dS tiles
    (the minimum ctattn_bwd accepts) recomputes S and dP instead.  Both against the oracle, and
    one byte less than the minimum is refused."""
    b, h, t, d = shape
    q, k, v, do = ora.make_inputs(shape, 77, std=0.5, dtype=fmt)
    td, code = (torch.bfloat16, 1) if fmt == "bf16" else (torch.float16, 2)
    say(f"dS / recompute paths shape={shape} causal={causal} {fmt}")
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(td)
                       for a in (q, k, v, do))
    o, lse = ct.flash_attn_fwd(tq, tk, tv, causal)
    full = ct._capi.bwd_workspace_bytes(td, b, h, t, d, causal, fastest=True)
    nt = (t + 31) // 32
    ds_bytes = b * h * (nt * (nt + 1) // 2 if causal else nt * nt) * 2048
    lib = ct._capi.load()
    want = ora.attention_fwd_bwd(q, k, v, do, causal)
    f = lambda x: x.float().cpu().numpy().astype(np.float64)  # noqa: E731
    for label, nbytes in (("dS", full), ("recompute", full - ds_bytes)):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        dq, dk, dv = (torch.empty_like(tq) for _ in range(3))
        rc = lib.ctattn_bwd(code, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), tdo.data_ptr(),
                            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), nbytes,
                            b, h, t, d, int(causal), None)
        assert rc == 0, ct._capi.last_error()
        torch.cuda.synchronize()
        got = {"o": f(o), "lse": f(lse), "dq": f(dq), "dk": f(dk), "dv": f(dv)}
        assert_close(got, want, "bf16", f"{shape} causal={causal} {fmt} {label}")
    ws = torch.empty(full - ds_bytes - 1, dtype=torch.uint8, device=DEV)
    rc = lib.ctattn_bwd(code, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), tdo.data_ptr(),
                        lse.data_ptr(), tq.data_ptr(), tq.data_ptr(), tq.data_ptr(), ws.data_ptr(),
                        full - ds_bytes - 1, b, h, t, d, int(causal), None)
    assert rc != 0 and "workspace" in ct._capi.last_error()


def test_c4_ds_path_matches_recompute_path(c4_run):
    """Config 4 at full size through the recomputing dQ kernel (the default workspace, which
    at this shape holds no dS tiles) against the fastest-workspace run (dS stored by the dK/dV
    kernel): dK and dV come from the
    same dK/dV kernel and agree bitwise; dQ agrees to bf16 rounding of dS (2e-2 of max |dQ| per
    head), and two heads of the recompute run against the oracle."""
    q, k, v, do, got = c4_run
    b, h, t, d = C4_SHAPE
    say("c4 full size bf16, recompute path")
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)
                       for a in (q, k, v, do))
    o, lse = ct.flash_attn_fwd(tq, tk, tv, True)
    nt = (t + 31) // 32
    nbytes = ct._capi.bwd_workspace_bytes(torch.bfloat16, b, h, t, d, True)
    assert nbytes == ct._capi.bwd_workspace_bytes(torch.bfloat16, b, h, t, d, True, fastest=True) - \
        b * h * nt * (nt + 1) // 2 * 2048
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    dq, dk, dv = (torch.empty_like(tq) for _ in range(3))
    rc = ct._capi.load().ctattn_bwd(1, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), tdo.data_ptr(),
                                    lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                                    nbytes, b, h, t, d, 1, None)
    assert rc == 0, ct._capi.last_error()
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy().astype(np.float64)  # noqa: E731
    rec = {"o": f(o), "lse": f(lse), "dq": f(dq), "dk": f(dk), "dv": f(dv)}
    assert np.array_equal(rec["dk"], got["dk"]) and np.array_equal(rec["dv"], got["dv"])
    diff = np.max(np.abs(rec["dq"] - got["dq"]), axis=(2, 3))
    scale = np.max(np.abs(got["dq"]), axis=(2, 3))
    assert np.all(diff <= 2e-2 * scale), f"dQ paths differ: {(diff / scale).max():.3e}"
    for hh in (3, 29):
        sl = lambda a: a[:, hh:hh + 1]  # noqa: E731
        want = ora.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), True, chunk_heads=1)
        assert_close({kk: sl(vv) for kk, vv in rec.items()}, want, "bf16", f"c4 recompute head {hh}")
