"""Pins the oracle against the reference's own compiled op: the committed golden vectors
(tests/golden/converse2d_ref.npz, written by tests/golden/make_golden.py from oracle/_ref) and, when
oracle/_ref is built, a live comparison in a subprocess on fresh random cases."""
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import converse_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLD = os.path.join(HERE, "golden", "converse2d_ref.npz")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "converse2d_ref.so")
MODES = ["constant", "reflect", "replicate", "circular"]


def golden_cases():
    g = np.load(GOLD)
    for i in range(int(g["ncases"])):
        B, C, H, W, k, s, p, m, pb = (int(v) for v in g[f"c{i}_meta"])
        yield (i, dict(x=g[f"c{i}_x"], w=g[f"c{i}_w"], b=g[f"c{i}_b"], s=s, p=p, mode=MODES[m],
                       eps=float(g[f"c{i}_eps"]), out64=g[f"c{i}_out64"], out32=g[f"c{i}_out32"]))


@pytest.mark.parametrize("i,case", list(golden_cases()))
def test_oracle_matches_reference_golden(i, case):
    got = O.converse2d_module(case["x"], case["w"], case["b"], case["s"], case["p"], case["mode"], case["eps"])
    # fp64 reference vs fp64 oracle: both divide by lambda in the same order
    np.testing.assert_allclose(got, case["out64"], atol=1e-9)
    # the reference's own fp32 result is within its documented cancellation error of the truth
    assert np.abs(case["out32"] - case["out64"]).max() < 5e-3


def test_oracle_matches_reference_golden_op_level():
    g = np.load(GOLD)
    for j in range(int(g["nops"])):
        got = O.converse2d_op(g[f"op{j}_x"], g[f"op{j}_x0"], g[f"op{j}_w"], g[f"op{j}_b"], int(g[f"op{j}_s"]), 1e-5)
        np.testing.assert_allclose(got, g[f"op{j}_out64"], atol=1e-9)


LIVE = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
torch.ops.load_library(sys.argv[2])
from oracle import converse_oracle as O
rng = np.random.default_rng(123)
worst = 0.0
for (B, C, h, w, k, s) in [(2, 3, 12, 14, 3, 1), (1, 2, 10, 9, 5, 2), (1, 2, 8, 10, 4, 3), (2, 1, 7, 7, 2, 4)]:
    x = rng.standard_normal((B, C, h, w)); x0 = rng.standard_normal((B, C, h * s, w * s))
    wt = rng.random((1, C, k, k)); wt /= wt.sum(axis=(2, 3), keepdims=True); b = rng.standard_normal((1, C, 1, 1))
    ref = torch.ops.converse2d.forward(*(torch.from_numpy(a) for a in (x, x0, wt, b)), s, 1e-5).numpy()
    worst = max(worst, float(np.abs(ref - O.converse2d_op(x, x0, wt, b, s, 1e-5)).max()))
print(worst)
"""


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built (make -C oracle)")
def test_oracle_matches_live_reference_op():
    r = subprocess.run([sys.executable, "-c", LIVE, ROOT, REF_SO], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert float(r.stdout.strip().splitlines()[-1]) < 1e-9
