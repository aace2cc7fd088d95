"""C-ABI boundary checks that need no GPU (CPU only).

libctattn.so must load and export every function include/ctattn.h declares, and the
host-side validation of every entry point must reject bad arguments before any HIP call
(so these run in a container without a GPU).
"""
import ctypes
import os
import subprocess

import pytest

from cudatransformer_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_capi.LIB_PATH):
        subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "cudatransformer_amd", "csrc")],
                       check=True)
    return _capi.load()


def test_exports_every_declared_symbol(lib):
    names = _capi.header_functions()
    assert set(names) >= {"ctattn_fwd", "ctattn_bwd", "ctattn_bwd_workspace_bytes",
                          "ctattn_last_error", "ctattn_set_policy", "ctattn_get_policy",
                          "ctattn_version"}
    raw = ctypes.CDLL(_capi.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in include/ctattn.h but not exported"


def _header_arity() -> dict:
    """Parameter count of every function include/ctattn.h declares."""
    import re
    text = re.sub(r"/\*.*?\*/", "", open(_capi.HEADER_PATH).read(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(ctattn_\w+)\s*\(([^)]*)\)", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_header(lib):
    """Every ctypes signature the Python binding declares has the header's parameter count."""
    arity = _header_arity()
    assert set(arity) == set(_capi.header_functions())
    for name, n in arity.items():
        argtypes = getattr(lib, name).argtypes
        assert argtypes is not None, f"{name}: no ctypes signature"
        assert len(argtypes) == n, f"{name}: ctypes declares {len(argtypes)} parameters, header {n}"


def test_exports_nothing_else(lib):
    """The library is built with hidden visibility: its dynamic symbol table defines exactly
    the functions the header declares (internal C++ symbols stay private, so two builds
    loaded in one process cannot interpose on each other)."""
    nm = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True,
                        text=True)
    if nm.returncode != 0:
        pytest.skip("nm unavailable")
    funcs = {line.split()[-1] for line in nm.stdout.splitlines()
             if len(line.split()) == 3 and line.split()[1] == "T"}
    assert funcs == set(_capi.header_functions())


def test_version(lib):
    assert lib.ctattn_version() == 200


def test_bad_dtype_rejected(lib):
    rc = lib.ctattn_fwd(7, 1, 1, 1, 1, None, 1, 1, 8, 64, 0, None)
    assert rc == 1  # hipErrorInvalidValue
    assert "unknown dtype" in _capi.last_error()


@pytest.mark.parametrize("d", [0, 257, 1024])
def test_bad_head_dim_rejected(lib, d):
    rc = lib.ctattn_fwd(0, 1, 1, 1, 1, None, 1, 1, 8, d, 0, None)
    assert rc == 801  # hipErrorNotSupported
    assert "head dim" in _capi.last_error()


def test_negative_size_rejected(lib):
    assert lib.ctattn_fwd(0, 1, 1, 1, 1, None, -1, 1, 8, 64, 0, None) == 1
    assert lib.ctattn_bwd_workspace_bytes(0, 1, -3, 8, 64, 1) == -1


def test_too_many_rows_rejected(lib):
    assert lib.ctattn_fwd(0, 1, 1, 1, 1, None, 1 << 16, 1 << 10, 1 << 10, 64, 0, None) == 1
    assert "2^31" in _capi.last_error()


def test_null_pointers_rejected(lib):
    assert lib.ctattn_fwd(0, None, 1, 1, 1, None, 1, 1, 8, 64, 0, None) == 1
    assert "null" in _capi.last_error()
    assert lib.ctattn_bwd(0, 1, 1, 1, 1, 1, None, 1, 1, 1, 1, 1 << 20, 1, 1, 8, 64, 0, None) == 1


def test_empty_problem_is_a_noop(lib):
    # No element to compute: success without touching the GPU (there is none here).
    assert lib.ctattn_fwd(0, None, None, None, None, None, 0, 4, 16, 64, 1, None) == 0
    assert lib.ctattn_fwd(1, None, None, None, None, None, 2, 4, 0, 64, 0, None) == 0
    assert lib.ctattn_last_error() == b""


def test_workspace_size_and_check(lib):
    prev = _capi.set_policy(_capi.POLICY_GENERIC)
    try:
        n = lib.ctattn_bwd_workspace_bytes(0, 2, 3, 100, 48, 1)
        assert n == ((2 * 3 * 100 * 4 + 255) // 256) * 256
        rc = lib.ctattn_bwd(0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, n - 1, 2, 3, 100, 48, 1, None)
        assert rc == 1 and "workspace" in _capi.last_error()
    finally:
        _capi.set_policy(prev)
    n_auto = lib.ctattn_bwd_workspace_bytes(0, 8, 12, 1024, 64, 1)
    assert n_auto >= 8 * 12 * 1024 * 4


def test_policy_roundtrip(lib):
    prev = _capi.set_policy(_capi.POLICY_GENERIC)
    assert lib.ctattn_get_policy() == _capi.POLICY_GENERIC
    _capi.set_policy(prev)
    assert lib.ctattn_get_policy() == prev
    prev = _capi.set_policy(_capi.POLICY_DETERMINISTIC)
    assert lib.ctattn_get_policy() == _capi.POLICY_DETERMINISTIC
    _capi.set_policy(prev)
    with pytest.raises(ValueError):
        _capi.set_policy(5)


def test_padded_head_dim_workspace(lib):
    """A head dim without its own MFMA kernel (d <= 128, not 32 / 64 / 128) runs padded to the
    next width: the backward workspace holds delta, the padded shape's MFMA scratch and eight
    padded copies (q, k, v, o, dO, dQ, dK, dV); d = 64 needs delta only (fp32, AUTO), and a
    head dim above 128 (generic kernels) as well."""
    def al(x):
        return (x + 255) // 256 * 256

    b, h, t = 2, 3, 150
    rows = b * h * t
    assert lib.ctattn_bwd_workspace_bytes(0, b, h, t, 64, 1) == al(rows * 4)
    for d, dp, eb, dtype in [(80, 128, 4, 0), (48, 64, 2, 1), (20, 32, 2, 2), (100, 128, 8, 3)]:
        stat = 8 if dtype == 3 else 4
        extra = al(rows * 4) if dtype in (1, 2) else 0  # bf16 / fp16: -LSE log2(e) per row
        want = al(rows * stat) + extra + 8 * al(rows * dp * eb)
        assert lib.ctattn_bwd_workspace_bytes(dtype, b, h, t, d, 1) == want, (d, dtype)
    assert lib.ctattn_bwd_workspace_bytes(0, b, h, t, 160, 1) == al(rows * 4)
    prev = _capi.set_policy(_capi.POLICY_GENERIC)
    try:
        assert lib.ctattn_bwd_workspace_bytes(0, b, h, t, 80, 1) == al(rows * 4)
    finally:
        _capi.set_policy(prev)


def test_deterministic_workspace_stays_linear(lib):
    """DETERMINISTIC fp32: dQ partials per 128-key block (one fp32 [B, H, T, d] plane each)
    while T <= 1024, none beyond (the query-major dQ kernel); the dS tiles (d >= 64) in their
    room while they add at most 2 x (q + k + v).  So the workspace is at most AUTO's plus 8 dQ
    planes plus 24 bytes per row element -- linear in B*H*T at every T.  AUTO needs delta only
    (d <= 64; its dS tiles are never in the default at these shapes)."""
    for shape in [(8, 12, 1024, 64), (2, 4, 1000, 32), (1, 32, 1025, 128), (1, 32, 131072, 128),
                  (16, 32, 32768, 64)]:
        b, h, t, d = shape
        rows_bytes = ((b * h * t * 4 + 255) // 256) * 256
        nkb = (t + 127) // 128
        partials = ((nkb * b * h * t * d * 4 + 255) // 256) * 256 if nkb <= 8 else 0
        sizes = {}
        for pol in (_capi.POLICY_AUTO, _capi.POLICY_DETERMINISTIC):
            prev = _capi.set_policy(pol)
            try:
                sizes[pol] = lib.ctattn_bwd_workspace_bytes(0, b, h, t, d, 1)
            finally:
                _capi.set_policy(prev)
        assert sizes[_capi.POLICY_AUTO] == rows_bytes, (shape, sizes)
        n64 = (t + 63) // 64
        ds = b * h * n64 * (n64 + 1) // 2 * 16384 if d >= 64 and t <= 32768 else 0
        ds = ds if ds <= 4 << 30 else 0
        room = ((max(partials, ds) + 255) // 256) * 256
        with_ds = room - partials <= 2 * 3 * b * h * t * d * 4
        assert sizes[_capi.POLICY_DETERMINISTIC] == rows_bytes + (room if with_ds else partials), (shape, sizes)
        assert sizes[_capi.POLICY_DETERMINISTIC] <= rows_bytes + (8 + 24) * b * h * t * d * 4


def test_no_gpu_call_raises_cleanly(lib):
    """Without a GPU a real compute call must fail with a message, never crash."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("GPU present: covered by the GPU tests")
    rc = lib.ctattn_fwd(0, 1, 1, 1, 1, None, 1, 1, 8, 64, 0, None)
    assert rc != 0
    assert _capi.last_error() != ""


def test_row_limit_boundary(lib):
    """B*H*T up to 2^31 - 1 rows is accepted on the host (the kernels loop over rows with a
    grid stride, so no launch exceeds 2^32 work-items); one row more is rejected."""
    assert lib.ctattn_bwd_workspace_bytes(0, 1, 1, 2 ** 31 - 1, 8, 0) >= (2 ** 31 - 1) * 4
    assert lib.ctattn_bwd_workspace_bytes(0, 1, 1, 2 ** 31, 8, 0) == -1
    assert lib.ctattn_bwd_workspace_bytes(1, 1 << 16, 1 << 5, 1 << 10, 128, 1) == -1


def test_bf16_ds_workspace(lib):
    """bf16 / fp16 at d = 128: ctattn_bwd_workspace_bytes_max asks for the dS tiles (2 KiB per
    32 x 32 tile of the mask: a triangle when causal) on top of delta and -LSE log2(e); other
    head dims do not, and above 4 GiB of tiles (or T > 65536) it stays linear in rows.
    The default ctattn_bwd_workspace_bytes includes the tiles only while they take at most
    twice the bytes of q, k and v."""
    def al(x):
        return (x + 255) // 256 * 256

    for (b, h, t) in [(1, 32, 8192), (2, 3, 333)]:
        rows, nt = b * h * t, (t + 31) // 32
        base = al(rows * 4) + al(rows * 4)
        for causal, tiles in ((1, nt * (nt + 1) // 2), (0, nt * nt)):
            for dtype in (1, 2):
                ds = b * h * tiles * 2048
                assert lib.ctattn_bwd_workspace_bytes_max(dtype, b, h, t, 128, causal) == base + ds
                in_default = ds <= 2 * 3 * rows * 128 * 2
                assert in_default == (t == 333)
                assert lib.ctattn_bwd_workspace_bytes(dtype, b, h, t, 128, causal) == base + (ds if in_default else 0)
            for fn in (lib.ctattn_bwd_workspace_bytes, lib.ctattn_bwd_workspace_bytes_max):
                assert fn(1, b, h, t, 64, causal) == base
    # B1 H32 T16384 causal: 8.6 GB of tiles, above the 4 GiB limit.
    assert lib.ctattn_bwd_workspace_bytes_max(1, 1, 32, 16384, 128, 1) == 2 * al(32 * 16384 * 4)
    assert lib.ctattn_bwd_workspace_bytes_max(1, 1, 1, 1 << 20, 128, 1) == 2 * al((1 << 20) * 4)


def test_f32_ds_workspace(lib):
    """fp32 dS tiles (16 KiB per 64 x 64 tile of the mask, a triangle when causal), asked for by
    ctattn_bwd_workspace_bytes_max where the policy takes the dS path: DETERMINISTIC at d in
    {64, 128} (in the room of the dQ partials, one plane per 128-key block up to T = 1024,
    whichever is larger); AUTO only at d = 128 on grids of at least 1024 key blocks of 64.
    Never at d = 32, nor above 4 GiB of tiles.  The default includes them only while the bytes
    they add take at most twice the bytes of q, k and v."""
    def al(x):
        return (x + 255) // 256 * 256

    for (b, h, t) in [(8, 12, 1024), (2, 3, 333), (1, 2, 64), (2, 64, 512)]:
        rows, n = b * h * t, (t + 63) // 64
        for causal, tiles in ((1, n * (n + 1) // 2), (0, n * n)):
            for d in (64, 128):
                ds = b * h * tiles * 16384
                in_default = ds <= 2 * 3 * rows * d * 4
                auto_ds = d == 128 and n * b * h >= 1024
                want_max = al(rows * 4) + (al(ds) if auto_ds else 0)
                assert lib.ctattn_bwd_workspace_bytes_max(0, b, h, t, d, causal) == want_max
                want = al(rows * 4) + (al(ds) if auto_ds and in_default else 0)
                assert lib.ctattn_bwd_workspace_bytes(0, b, h, t, d, causal) == want
                prev = _capi.set_policy(_capi.POLICY_DETERMINISTIC)
                try:
                    planes = -(-t // 128) * rows * d * 4 if t <= 1024 else 0
                    assert lib.ctattn_bwd_workspace_bytes_max(0, b, h, t, d, causal) == al(rows * 4) + al(max(planes, ds))
                    adds = al(max(planes, ds)) - al(planes)
                    want = al(rows * 4) + (al(max(planes, ds)) if adds <= 2 * 3 * rows * d * 4 else al(planes))
                    assert lib.ctattn_bwd_workspace_bytes(0, b, h, t, d, causal) == want
                finally:
                    _capi.set_policy(prev)
            for fn in (lib.ctattn_bwd_workspace_bytes, lib.ctattn_bwd_workspace_bytes_max):
                assert fn(0, b, h, t, 32, causal) == al(rows * 4)
    # B1 H32 T8192 d128 causal: 4.3 GB of tiles, above the 4 GiB limit.
    prev = _capi.set_policy(_capi.POLICY_DETERMINISTIC)
    try:
        assert lib.ctattn_bwd_workspace_bytes_max(0, 1, 32, 8192, 128, 1) == al(32 * 8192 * 4)
    finally:
        _capi.set_policy(prev)


def test_default_bwd_workspace_is_linear_in_rows(lib):
    """The default backward workspace grows linearly with B * H * T at every T, like the
    reference's backward memory (which never holds a T x T object): at most 8 bytes per row
    of statistics plus, while they are included, dS tiles of at most 2 x (q + k + v) =
    1536 bytes per row at bf16 d = 128 (fp32: 1536 at d = 64, 3072 at d = 128), plus alignment.
    B1 H32 T32768 d128 bf16 included."""
    for dtype, d, per_row in ((1, 128, 1536), (2, 128, 1536), (0, 64, 1536), (0, 128, 3072)):
        for causal in (0, 1):
            for t in [64, 128, 333, 1024, 1536, 2048, 4096, 8192, 16384, 32768, 65536]:
                rows = 32 * t
                n = lib.ctattn_bwd_workspace_bytes(dtype, 1, 32, t, d, causal)
                assert 0 < n <= rows * (8 + per_row) + 512, (dtype, causal, t, n)
                assert n <= lib.ctattn_bwd_workspace_bytes_max(dtype, 1, 32, t, d, causal)
    assert lib.ctattn_bwd_workspace_bytes(1, 1, 32, 32768, 128, 1) <= 32 * 32768 * 8 + 512


def test_fwd_workspace_bytes(lib):
    """The forward needs a workspace only for head dims that run padded: four [B,H,T,dp]
    copies (q, k, v, o), each 256-byte aligned; none for 32 / 64 / 128 or above 128."""
    def al(x):
        return (x + 255) // 256 * 256

    b, h, t = 2, 3, 100
    rows = b * h * t
    for d in (32, 64, 128, 160):
        assert lib.ctattn_fwd_workspace_bytes(0, b, h, t, d) == 0
    assert lib.ctattn_fwd_workspace_bytes(0, b, h, t, 48) == 4 * al(rows * 64 * 4)
    assert lib.ctattn_fwd_workspace_bytes(1, b, h, t, 80) == 4 * al(rows * 128 * 2)
    assert lib.ctattn_fwd_workspace_bytes(3, b, h, t, 16) == 4 * al(rows * 32 * 8)
    assert lib.ctattn_fwd_workspace_bytes(0, b, -1, t, 48) == -1
    prev = _capi.set_policy(_capi.POLICY_GENERIC)
    try:
        assert lib.ctattn_fwd_workspace_bytes(0, b, h, t, 48) == 0
    finally:
        _capi.set_policy(prev)