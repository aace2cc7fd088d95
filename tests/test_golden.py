"""Golden fixtures (tests/golden/*.npz) are reproduced by both oracle restatements (CPU)."""
import glob
import os

import numpy as np
import pytest

from oracle import attention_fp64 as ora
from oracle import c_oracle

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def test_fixtures_present():
    names = {os.path.basename(p) for p in GOLDEN}
    assert "c1_b1h4t128d32_f32.npz" in names and len(names) >= 5


@pytest.mark.parametrize("path", GOLDEN, ids=os.path.basename)
@pytest.mark.parametrize("causal", [False, True])
def test_oracles_reproduce_fixture(path, causal):
    import subprocess

    subprocess.run(["make", "-s", "-C", os.path.dirname(c_oracle.__file__)], check=True)
    z = np.load(path)
    tag = "causal" if causal else "full"
    dense = ora.attention_fwd_bwd(z["q"], z["k"], z["v"], z["do"], causal)
    o, lse = c_oracle.fwd(z["q"], z["k"], z["v"], causal)
    dq, dk, dv = c_oracle.bwd(z["q"], z["k"], z["v"], o, z["do"], lse, causal)
    online = {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}
    for key in ("o", "lse", "dq", "dk", "dv"):
        want = z[f"{key}_{tag}"]
        scale = max(1.0, float(np.max(np.abs(want))))
        assert np.max(np.abs(dense[key] - want)) <= 1e-6 * scale, key
        assert np.max(np.abs(online[key] - want)) <= 1e-6 * scale, key


def test_c1_fixture_matches_its_recipe():
    """c1 = B1 H4 T128 d32, N(0,1), seed 1, drawn Q, K, V, dO in fp64 then cast to fp32."""
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_b1h4t128d32_f32.npz"))
    q, k, v, do = ora.make_inputs((1, 4, 128, 32), seed=1)
    for name, a in (("q", q), ("k", k), ("v", v), ("do", do)):
        assert np.array_equal(z[name], a), name
