"""Model parity at the benchmark's own batch sizes, and trained-lambda layers, on the GPU.

cfg4: Converse-DnCNN (models/converse_dncnn.py:11-35) at B = 8, the batch bench.py times; every image
against the fp64 oracle.  cfg5: Converse-USRNet (models/converse_usrnet.py:178-214) at B = 4 with
KernelNet(25) and non-zero alphas; every image against the fp64 oracle.  Each model's forward is
recorded call by call (route, scratch) so the tests also assert that the kernels the benchmark times
are the ones that ran: the 268 path for every DnCNN layer; for USRNet one workgroup per plane (no
split scratch) on the 260 x 260 body planes (512 planes) and the 256 x 256 data steps (256 planes),
the generic passes for the s = 4 data step.  Gate (north star): PSNR >= 60 dB against the oracle,
peak = dynamic range of the oracle output.

Trained lambda: the psf and bias of the smallest-lambda Converse2D layer of each shipped checkpoint
(tests/golden/trained_layers.npz, written by tests/golden/make_trained_layers.py) at its model's layer
shape, against the fp64 oracle at max-abs <= 1e-4.
"""
import os

import numpy as np
import pytest
import torch

import bench
from conversenet_amd import _lib
from conversenet_amd import functional as Fh
from oracle import converse_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "trained_layers.npz")


def _sd(m):
    return {k: v.detach().cpu().numpy() for k, v in m.state_dict().items()}


def psnr(a, ref):
    mse = float(np.mean((a.astype(np.float64) - ref) ** 2))
    return 10 * np.log10((ref.max() - ref.min()) ** 2 / mse) if mse > 0 else np.inf


def _run_recording(fn):
    """Runs fn() and returns (its result, [(geometry, (route, table bytes, scratch bytes)), ...]) for
    every module-level Converse2D call it made (functional.converse2d_fused, the library's plan for
    that geometry)."""
    import inspect
    calls = []
    orig = Fh.converse2d_fused
    sig = inspect.signature(orig)

    def rec(*args, **kw):
        a = sig.bind(*args, **kw)
        a.apply_defaults()
        x, w = a.arguments["x"], a.arguments["weight"]
        geo = (*(int(v) for v in x.shape), int(w.shape[0]), int(w.shape[2]), int(w.shape[3]),
               int(a.arguments["scale"]), int(a.arguments["padding"]))
        calls.append((geo, Fh._module_plan(_lib.load(), *geo)))
        return orig(*args, **kw)

    Fh.converse2d_fused = rec
    try:
        with torch.no_grad():
            out = fn()
        torch.cuda.synchronize()
    finally:
        Fh.converse2d_fused = orig
    return out, calls


@pytest.fixture(scope="module")
def dncnn_b8():
    m, x = bench.make_dncnn(torch, DEV, batch=8)
    got, calls = _run_recording(lambda: m(x).cpu().numpy())
    return _sd(m), x.cpu().numpy(), got, calls


def test_converse_dncnn_b8_routes(dncnn_b8):
    _, x, got, calls = dncnn_b8
    assert x.shape == (8, 1, 256, 256) and got.shape == (8, 1, 256, 256)
    assert len(calls) == 20
    for geo, (route, _, _) in calls:  # the 268 path's scratch holds its half spectra between passes
        assert geo == (8, 128, 256, 256, 1, 7, 7, 1, 6) and route == _lib.ROUTE_PFA268


@pytest.mark.parametrize("i", range(8))
def test_converse_dncnn_b8_image(dncnn_b8, i):
    sd, x, got, _ = dncnn_b8
    ref = O.converse_dncnn(x[i:i + 1], sd)
    p = psnr(got[i:i + 1], ref)
    print(f"cfg4 Converse-DnCNN B8 image {i}: PSNR {p:.1f} dB, max-abs {np.abs(got[i:i + 1] - ref).max():.3e}, "
          f"|ref| max {np.abs(ref).max():.3f}")
    assert p >= 60


@pytest.fixture(scope="module")
def usrnet_b4():
    m, x, k = bench.make_usrnet(torch, DEV, batch=4)
    got, calls = _run_recording(lambda: m(x, k, 4).cpu().numpy())
    return _sd(m), x.cpu().numpy(), k.cpu().numpy(), got, calls


def test_converse_usrnet_b4_routes(usrnet_b4):
    _, x, k, got, calls = usrnet_b4
    assert x.shape == (4, 3, 64, 64) and k.shape == (4, 1, 25, 25) and got.shape == (4, 3, 256, 256)
    body = (4, 128, 256, 256, 1, 3, 3, 1, 2)
    step0 = (4, 64, 64, 64, 4, 25, 25, 4, 0)
    steps = (4, 64, 256, 256, 4, 25, 25, 1, 0)
    seen = [geo for geo, _ in calls]
    assert seen.count(body) == 35 and seen.count(step0) == 1 and seen.count(steps) == 4 and len(seen) == 40
    for geo, (route, _, sb) in calls:  # one 1024-thread workgroup per plane: no split scratch requested
        assert route == _lib.ROUTE_FUSED and sb == 0


@pytest.mark.parametrize("i", range(4))
def test_converse_usrnet_b4_image(usrnet_b4, i):
    sd, x, k, got, _ = usrnet_b4
    ref = O.converse_usrnet(x[i:i + 1], k[i:i + 1], 4, sd, 25)
    p = psnr(got[i:i + 1], ref)
    print(f"cfg5 Converse-USRNet B4 image {i}: PSNR {p:.1f} dB, max-abs {np.abs(got[i:i + 1] - ref).max():.3e}, "
          f"|ref| max {np.abs(ref).max():.3f}")
    assert p >= 60


# (checkpoint, layer shape B, C, H, W, k, padding, mode, route): the trained layer at its model's shape
TRAINED = [
    ("converse_dncnn", (8, 128, 256, 256), 7, 6, "circular", _lib.ROUTE_PFA268),
    ("converse_usrnet", (4, 128, 256, 256), 3, 2, "circular", _lib.ROUTE_FUSED),
    ("converse_srresnet", (1, 128, 128, 128), 5, 4, "replicate", _lib.ROUTE_GENERIC),
]


@pytest.mark.parametrize("name,shape,k,p,mode,route", TRAINED, ids=[t[0] for t in TRAINED])
def test_trained_lambda_layer(name, shape, k, p, mode, route):
    """A trained psf and bias (smallest lambda of the checkpoint) at the model's layer shape.  The input
    is N(0,1); the oracle runs one batch element at a time (host memory)."""
    g = np.load(GOLDEN, allow_pickle=False)
    w, b = g[f"{name}.weight"], g[f"{name}.bias"]
    assert w.shape == (1, shape[1], k, k)
    lam = 1 / (1 + np.exp(-(b.astype(np.float64) - 9))) + 1e-5
    assert abs(lam.min() - float(g[f"{name}.lambda_min"])) < 1e-9
    rng = np.random.default_rng(17)
    x = rng.standard_normal(shape).astype(np.float32)
    xd, wd, bd = (torch.from_numpy(a).to(DEV) for a in (x, w, b))
    assert Fh.module_route(shape, wd, 1, p) == route
    got = Fh.converse2d_fused(xd, wd, bd.reshape(-1), 1, p, mode, 1e-5).cpu().numpy()
    err = 0.0
    for i in range(shape[0]):
        ref = O.converse2d_module(x[i:i + 1], w, b, 1, p, mode, 1e-5)
        err = max(err, float(np.abs(got[i:i + 1] - ref).max()))
    print(f"trained {name} ({g[f'{name}.layer']}, lambda min {lam.min():.3e}) {shape} k{k} p{p} {mode}: "
          f"max-abs {err:.3e}")
    assert err <= 1e-4
