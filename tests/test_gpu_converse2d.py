"""HIP Converse2D forward vs the fp64 oracle (parity gate: max-abs <= 1e-4)."""
import itertools

import numpy as np
import pytest
import torch

from oracle import converse_oracle as O
from tests.conftest import seeded, softmax_psf

pytestmark = pytest.mark.gpu
TOL = 1e-4

MODES = ["circular", "reflect", "replicate", "constant"]


def _run_fused(x, w, b, s, p, mode, eps):
    from conversenet_amd import functional as Fh
    dev = torch.device("cuda")
    out = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                              torch.from_numpy(b).reshape(-1).to(dev), s, p, mode, eps)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# the reference's test_error.py grid (B, C, H, W, k, s), padding k // 2, circular
GRID = list(itertools.product([1, 2], [2, 3], [16, 32], [18, 40], [3, 5], [1, 2, 3]))


@pytest.mark.parametrize("B,C,H,W,k,s", GRID)
def test_reference_grid(B, C, H, W, k, s):
    rng = seeded(B, C, H, W, k, s)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, s, k // 2, "circular", 1e-5)
    got = _run_fused(x, w, b, s, k // 2, "circular", 1e-5)
    assert got.shape == ref.shape
    err = np.abs(got - ref).max()
    assert err <= TOL, err


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("s", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [2, 3, 4, 5, 7])
def test_padding_modes_scales_kernels(mode, s, k):
    rng = np.random.default_rng(1000 + 10 * s + k)
    H, W = 13, 17
    p = min(k - 1, 4)
    x = rng.standard_normal((2, 3, H, W)).astype(np.float32)
    w = softmax_psf(rng, 3, k)
    b = (0.5 * rng.standard_normal((1, 3, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, s, p, mode, 1e-5)
    got = _run_fused(x, w, b, s, p, mode, 1e-5)
    assert np.abs(got - ref).max() <= TOL


def test_cfg1_shape():
    rng = np.random.default_rng(0)
    x = rng.random((1, 64, 128, 128), dtype=np.float32)
    w = softmax_psf(np.random.default_rng(1), 64, 5)
    b = np.zeros((1, 64, 1, 1), np.float32)
    ref = O.converse2d_module(x, w, b, 1, 2, "circular", 1e-5)
    got = _run_fused(x, w, b, 1, 2, "circular", 1e-5)
    err = np.abs(got - ref).max()
    print("cfg1 max-abs vs fp64 oracle:", err)
    assert err <= TOL


def test_cfg2_shape():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 64, 64, 64)).astype(np.float32)
    w = softmax_psf(np.random.default_rng(1), 64, 3)
    b = np.zeros((1, 64, 1, 1), np.float32)
    ref = O.converse2d_module(x, w, b, 2, 1, "circular", 1e-5)
    got = _run_fused(x, w, b, 2, 1, "circular", 1e-5)
    err = np.abs(got - ref).max()
    print("cfg2 max-abs vs fp64 oracle:", err)
    assert err <= TOL


@pytest.mark.parametrize("s", [1, 2, 3])
def test_op_level_arbitrary_x0(s):
    from conversenet_amd import functional as Fh
    rng = np.random.default_rng(7 + s)
    B, C, h, w, k = 2, 3, 20, 22, 5
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_op(x, x0, wt, b, s, 1e-5)
    dev = torch.device("cuda")
    got = Fh.converse2d_op(*(torch.from_numpy(a).to(dev) for a in (x, x0, wt, b)), s, 1e-5).cpu().numpy()
    assert np.abs(got - ref).max() <= TOL


# ---------------------------------------------------------------------------------------------
# fused single-kernel path (scale 1, padded planes with an instantiated plan: 260x260, 132x132)
# ---------------------------------------------------------------------------------------------
FUSED_CASES = [
    # (B, C, H, W, k, p, mode)
    (2, 3, 256, 256, 5, 2, "circular"),
    (1, 2, 256, 256, 5, 2, "reflect"),
    (1, 2, 256, 256, 3, 2, "replicate"),
    (1, 2, 254, 254, 7, 3, "constant"),
    (1, 2, 248, 248, 9, 6, "circular"),
    (2, 3, 128, 128, 5, 2, "circular"),
    (1, 2, 130, 130, 3, 1, "reflect"),
    (1, 3, 124, 124, 4, 4, "replicate"),
]


@pytest.mark.parametrize("B,C,H,W,k,p,mode", FUSED_CASES)
def test_fused_path_vs_oracle(B, C, H, W, k, p, mode):
    rng = seeded("fused", B, C, H, W, k, p, mode)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, 1, p, mode, 1e-5)
    got = _run_fused(x, w, b, 1, p, mode, 1e-5)
    err = np.abs(got - ref).max()
    print(f"fused {H + 2 * p}^2 {mode} k{k}: max-abs {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("act", [None, "gelu"])
def test_fused_260_wide_rows_no_padding(act):
    """An already padded 260 x 260 plane with no padding to apply (the operator path's module route):
    the fused kernel takes the row tail past 256 columns through single-word loads and stores."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    rng = seeded("fused260", act)
    B, C, k = 2, 3, 5
    x = rng.standard_normal((B, C, 260, 260)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    assert _lib.load().cvn_converse2d_route(B, C, 260, 260, 1, k, k, 1, 0) == _lib.ROUTE_FUSED
    ref = O.converse2d_module(x, w, b, 1, 0, "constant", 1e-5)
    if act:
        ref = O.gelu(ref)
    dev = torch.device("cuda")
    got = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                              torch.from_numpy(b).reshape(-1).to(dev), 1, 0, "constant", 1e-5, act=act)
    err = np.abs(got.cpu().numpy() - ref).max()
    print(f"fused 260 wide, no padding, act {act}: max-abs {err:.3e}")
    assert err <= TOL, err


def test_fused_per_sample_psf_and_gelu():
    from conversenet_amd import functional as Fh
    rng = seeded("fused-ps")
    B, C, H, W, k = 2, 3, 256, 256, 5
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k, batch=B)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.gelu(O.converse2d_module(x, w, b, 1, 2, "circular", 1e-3))
    dev = torch.device("cuda")
    got = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                              torch.from_numpy(b).reshape(-1).to(dev), 1, 2, "circular", 1e-3, act="gelu")
    assert np.abs(got.cpu().numpy() - ref).max() <= TOL


def test_transfer_table_cache_follows_in_place_updates():
    """A cached table must not survive an in-place weight update (the reference's data_ptr-keyed
    OTF cache, converse2d.cpp:62-66, returns a stale OTF in that case)."""
    from conversenet_amd import functional as Fh
    dev = torch.device("cuda")
    rng = seeded("cache")
    x = torch.from_numpy(rng.standard_normal((1, 2, 128, 128)).astype(np.float32)).to(dev)
    w = torch.from_numpy(softmax_psf(rng, 2, 5)).to(dev)
    b = torch.zeros(2, device=dev)
    y1 = Fh.converse2d_fused(x, w, b, 1, 2, "circular", 1e-5)
    y1b = Fh.converse2d_fused(x, w, b, 1, 2, "circular", 1e-5)
    assert torch.equal(y1, y1b)
    with torch.no_grad():
        w.copy_(torch.from_numpy(softmax_psf(rng, 2, 5)).to(dev))  # same storage, new values
    y2 = Fh.converse2d_fused(x, w, b, 1, 2, "circular", 1e-5)
    ref = O.converse2d_module(x.cpu().numpy(), w.cpu().numpy(), b.reshape(1, 2, 1, 1).cpu().numpy(), 1, 2,
                              "circular", 1e-5)
    assert np.abs(y2.cpu().numpy() - ref).max() <= TOL
    torch.ops.converse2d.clear_cache()
    assert len(Fh.table_cache.entries) == 0


# 256 x 256 planes: the fused kernel's Cooley-Tukey plan (rows 16 x 16, columns 2 x 8 x 8 with twiddles)
CT256_CASES = [
    # B, C, H, p, mode, k, per-sample psf, act
    (2, 3, 256, 0, "circular", 5, False, None),
    (2, 4, 256, 0, "circular", 25, True, None),      # Converse-USRNet's data step (per-sample 25 x 25 psf)
    (1, 2, 252, 2, "reflect", 5, False, "gelu"),
    (1, 2, 240, 8, "replicate", 7, False, None),
    (1, 3, 248, 4, "constant", 9, True, "gelu"),
    (3, 2, 244, 6, "circular", 4, False, None),
]


@pytest.mark.parametrize("B,C,H,p,mode,k,ps,act", CT256_CASES)
def test_fused_256_cooley_tukey(B, C, H, p, mode, k, ps, act, monkeypatch):
    """256 x 256 padded planes on the fused route against the fp64 oracle and the generic passes."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    rng = seeded("ct256", B, C, H, p, mode, k, ps, act)
    x = rng.standard_normal((B, C, H, H)).astype(np.float32)
    w = softmax_psf(rng, C, k, batch=B if ps else 1)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    eps = 1e-3 if ps else 1e-5
    monkeypatch.delenv("CVN_DISABLE_FUSED", raising=False)
    assert _lib.load().cvn_converse2d_route(B, C, H, H, w.shape[0], k, k, 1, p) == _lib.ROUTE_FUSED
    ref = O.converse2d_module(x, w, b, 1, p, mode, eps)
    if act:
        ref = O.gelu(ref)
    dev = torch.device("cuda")

    def run():
        out = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                                  torch.from_numpy(b).reshape(-1).to(dev), 1, p, mode, eps, act=act)
        return out.cpu().numpy()

    fused = run()
    err = np.abs(fused - ref).max()
    print(f"fused 256^2 (Cooley-Tukey) B{B} C{C} p{p} {mode} k{k} per-sample {ps} act {act}: max-abs {err:.3e}")
    assert err <= TOL, err
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    generic = run()
    assert np.abs(fused - generic).max() <= TOL


SPLIT_CASES = [
    # B, C, H, p, mode, k, per-sample psf, act (padded sides 132, 256 and 260)
    (1, 5, 128, 2, "circular", 5, False, None),      # 5 planes: a partly filled block of 8
    (2, 64, 128, 2, "reflect", 3, False, "gelu"),    # 128 planes: the largest split
    (1, 129, 128, 2, "circular", 5, False, None),    # 129 planes: one workgroup per plane
    (3, 3, 252, 2, "replicate", 5, True, None),      # Cooley-Tukey 256 plan, per-sample psf
    (1, 130, 252, 2, "circular", 5, False, None),    # ... above the split limit
    (1, 9, 256, 2, "circular", 5, False, None),      # 260 plan
    (2, 3, 260, 0, "constant", 5, False, "gelu"),    # 260 plan, rows past 256 columns
]


@pytest.mark.parametrize("B,C,H,p,mode,k,ps,act", SPLIT_CASES)
def test_fused_split_small_plane_counts(B, C, H, p, mode, k, ps, act, monkeypatch):
    """At most 128 planes on the fused route: the route asks for scratch, and with it each plane's two
    row groups run in workgroups of their own (a forward kernel writing the group spectra, an inverse
    kernel combining them); given no scratch, the apply runs one workgroup per plane.  Both against the
    fp64 oracle, and against each other."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    lib = _lib.load()
    rng = seeded("split", B, C, H, p, mode, k, ps, act)
    x = rng.standard_normal((B, C, H, H)).astype(np.float32)
    w = softmax_psf(rng, C, k, batch=B if ps else 1)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    eps = 1e-3 if ps else 1e-5
    pb = w.shape[0]
    monkeypatch.delenv("CVN_DISABLE_FUSED", raising=False)
    geo = (B, C, H, H, pb, k, k, 1, p)
    assert lib.cvn_converse2d_route(*geo) == _lib.ROUTE_FUSED
    sb = lib.cvn_converse2d_scratch_bytes(*geo, _lib.ROUTE_FUSED)
    assert (sb > 0) == (B * C <= 128)
    ref = O.converse2d_module(x, w, b, 1, p, mode, eps)
    if act:
        ref = O.gelu(ref)
    dev = torch.device("cuda")
    xt, wt, bt = (torch.from_numpy(a).to(dev) for a in (x, w, b.reshape(-1)))
    split = Fh.converse2d_fused(xt, wt, bt, 1, p, mode, eps, act=act).cpu().numpy()
    tb = lib.cvn_converse2d_table_bytes(*geo, _lib.ROUTE_FUSED)
    table = torch.empty(tb, dtype=torch.uint8, device=dev)
    out = torch.empty_like(xt)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.cvn_converse2d_table_f32(wt.data_ptr(), pb, k, k, bt.data_ptr(), eps, B, C, H, H, 1, p,
                                        _lib.ROUTE_FUSED, table.data_ptr(), tb, st) == 0
    assert lib.cvn_converse2d_apply_f32(xt.data_ptr(), B, C, H, H, pb, k, k, 1, p, _lib.PAD_MODES[mode],
                                        _lib.ACT_GELU if act else _lib.ACT_NONE, _lib.ROUTE_FUSED,
                                        table.data_ptr(), tb, None, 0, out.data_ptr(), st) == 0
    whole = out.cpu().numpy()
    e_split, e_whole = np.abs(split - ref).max(), np.abs(whole - ref).max()
    print(f"fused {H + 2 * p}^2 B{B} C{C} {mode} k{k} per-sample {ps} act {act}: split {e_split:.3e}, "
          f"one workgroup per plane {e_whole:.3e}")
    assert e_split <= TOL and e_whole <= TOL
    assert np.abs(split - whole).max() <= 1e-5


@pytest.mark.parametrize("H,p", [(256, 2), (128, 2)])
def test_fused_matches_generic_path(H, p, monkeypatch):
    """The fused single-kernel path and the generic multi-pass path agree (both vs the oracle)."""
    rng = seeded("fvg", H, p)
    x = rng.standard_normal((2, 4, H, H)).astype(np.float32)
    w = softmax_psf(rng, 4, 5)
    b = (0.3 * rng.standard_normal((1, 4, 1, 1))).astype(np.float32)
    fused = _run_fused(x, w, b, 1, p, "circular", 1e-5)
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    generic = _run_fused(x, w, b, 1, p, "circular", 1e-5)
    ref = O.converse2d_module(x, w, b, 1, p, "circular", 1e-5)
    assert np.abs(fused - ref).max() <= TOL and np.abs(generic - ref).max() <= TOL
    assert np.abs(fused - generic).max() <= TOL


# ---------------------------------------------------------------------------------------------
# prime factors above 13 (Rader stages): 268 = 4*67 (cfg4's layer plane), 67, 17*19 (two Rader
# primes in one plan), 4*17*17 (a repeated Rader prime), 2*47 (generic O(R^2) stage), scale 2
# ---------------------------------------------------------------------------------------------
RADER_CASES = [
    # (B, C, H, W, k, s, p, mode)
    (1, 4, 256, 256, 7, 1, 6, "circular"),
    (2, 2, 61, 65, 5, 1, 3, "reflect"),
    (1, 2, 319, 315, 5, 1, 2, "circular"),
    (1, 1, 1152, 20, 5, 1, 2, "replicate"),
    (1, 2, 90, 40, 3, 1, 2, "constant"),
    (2, 2, 15, 19, 3, 2, 2, "circular"),
]


@pytest.mark.parametrize("B,C,H,W,k,s,p,mode", RADER_CASES)
def test_rader_prime_sizes(B, C, H, W, k, s, p, mode):
    rng = seeded("rader", B, C, H, W, k, s, p, mode)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, s, p, mode, 1e-5)
    got = _run_fused(x, w, b, s, p, mode, 1e-5)
    err = np.abs(got - ref).max()
    print(f"rader {H + 2 * p}x{W + 2 * p} s{s}: max-abs {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("s", [1, 2])
def test_rader_op_level(s):
    from conversenet_amd import functional as Fh
    rng = seeded("rader-op", s)
    B, C, h, w, k = 1, 2, 67, 38, 5
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_op(x, x0, wt, b, s, 1e-5)
    dev = torch.device("cuda")
    got = Fh.converse2d_op(*(torch.from_numpy(a).to(dev) for a in (x, x0, wt, b)), s, 1e-5).cpu().numpy()
    assert np.abs(got - ref).max() <= TOL


# ---------------------------------------------------------------------------------------------
# 268 x 268 planes (Converse-DnCNN: 256^2, padding 6): in-place prime-factor path 268 = 4 * 67
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("k", [7, 5])
def test_pfa268_vs_oracle(mode, k):
    rng = seeded("pfa268", mode, k)
    B, C, H, W = 2, 3, 256, 256
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, 1, 6, mode, 1e-5)
    got = _run_fused(x, w, b, 1, 6, mode, 1e-5)
    err = np.abs(got - ref).max()
    print(f"pfa268 {mode} k{k}: max-abs {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("H,p,k,mode", [(268, 0, 3, "constant"), (266, 1, 3, "reflect"), (264, 2, 5, "replicate")])
def test_pfa268_other_paddings(H, p, k, mode):
    """268-point planes reached with padding 0, 1, 2 (every padded column and row index map of the
    quad loads), 7 planes so the row pass's last block is partial."""
    rng = seeded("pfa268-pad", H, p, k, mode)
    B, C = 1, 7
    x = rng.standard_normal((B, C, H, H)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, 1, p, mode, 1e-5)
    got = _run_fused(x, w, b, 1, p, mode, 1e-5)
    assert np.abs(got - ref).max() <= TOL


def test_pfa268_per_sample_psf_gelu_and_generic_agreement(monkeypatch):
    from conversenet_amd import functional as Fh
    rng = seeded("pfa268-ps")
    B, C, H, W, k = 2, 2, 258, 258, 7
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k, batch=B)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.gelu(O.converse2d_module(x, w, b, 1, 5, "circular", 1e-3))
    dev = torch.device("cuda")
    args = (torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), torch.from_numpy(b).reshape(-1).to(dev), 1, 5,
            "circular", 1e-3)
    got = Fh.converse2d_fused(*args, act="gelu").cpu().numpy()
    assert np.abs(got - ref).max() <= TOL
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    generic = Fh.converse2d_fused(*args, act="gelu", cache=False).cpu().numpy()
    assert np.abs(got - generic).max() <= TOL


# ---------------------------------------------------------------------------------------------
# ConvReverseDataNet step (converse_usrnet.py:41-68): per-sample 25x25 psf of KernelNet scale (not
# normalised), eps 1e-3, padding 0; plane sides chosen so the transfer-table kernel runs partial
# column chunks, several rows per thread (Hs > 256) and every scale of the data steps.
# ---------------------------------------------------------------------------------------------
DATA_STEP_CASES = [
    # (B, C, h, w, s)
    (2, 5, 64, 64, 1),
    (2, 3, 256, 48, 1),
    (1, 2, 96, 80, 1),
    (2, 3, 300, 40, 1),
    (2, 4, 16, 16, 4),
    (1, 3, 64, 64, 4),
    (1, 2, 24, 20, 2),
    (2, 3, 30, 26, 2),
    (1, 2, 100, 34, 3),
]


@pytest.mark.parametrize("B,C,h,w,s", DATA_STEP_CASES)
def test_data_step_per_sample_psf(B, C, h, w, s):
    from conversenet_amd import functional as Fh
    rng = np.random.default_rng(1000 + 7 * s + h)
    x = rng.random((B, C, h, w)).astype(np.float32)
    k = (0.05 * rng.standard_normal((B, C, 25, 25))).astype(np.float32)
    alpha = (0.1 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.conv_reverse_datanet(x, k, s, alpha, 1e-3)
    dev = torch.device("cuda")
    got = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(k).to(dev),
                              torch.from_numpy(alpha).to(dev).reshape(-1), s, 0, "circular", 1e-3,
                              cache=False).cpu().numpy()
    err = np.abs(got - ref).max()
    print(f"data step B{B} C{C} {h}x{w} s{s}: max-abs {err:.3e} (|ref| max {np.abs(ref).max():.2f})")
    assert err <= TOL


# (B, C, h, w, s, k, x0): shapes the op path runs on compile-time plans (every planned row length and
# every (h, s) column plan at least once), then the reference's timing grid (test_speed.py:137-146,
# 253-271: B8 C8 256x256, x0 = nearest(x)) at s = 2 and 3
OP_PLANNED = [(1, 2, 64, 64, 2, 3, "rand"), (2, 3, 64, 128, 3, 5, "rand"), (1, 2, 128, 64, 4, 5, "rand"),
              (1, 1, 128, 192, 2, 7, "rand"), (2, 2, 256, 64, 2, 5, "rand"), (1, 2, 64, 256, 4, 3, "rand"),
              (1, 2, 256, 128, 3, 4, "rand"), (1, 2, 128, 128, 3, 6, "rand"), (1, 2, 64, 64, 3, 2, "rand"),
              (1, 2, 256, 256, 4, 5, "nearest"),
              (8, 8, 256, 256, 2, 5, "nearest"), (8, 8, 256, 256, 3, 3, "nearest"), (8, 8, 256, 256, 3, 7, "rand")]


@pytest.mark.parametrize("B,C,h,w,s,k,x0kind", OP_PLANNED)
def test_op_level_planned(B, C, h, w, s, k, x0kind):
    """converse2d::forward (converse2d.cpp:165-209) with arbitrary x0 on the compile-time-plan kernels,
    against the fp64 oracle (one batch element at a time), max-abs <= 1e-4."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    lib = _lib.load()
    assert lib.cvn_converse2d_op_route(h, w, s) == _lib.ROUTE_OP_PLANNED
    rng = seeded("op-planned", B, C, h, w, s, k, x0kind)
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    if x0kind == "nearest":
        x0 = np.repeat(np.repeat(x, s, axis=2), s, axis=3)
    else:
        x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    dev = torch.device("cuda")
    got = Fh.converse2d_op(*(torch.from_numpy(a).to(dev) for a in (x, x0, wt, b)), s, 1e-5).cpu().numpy()
    err = 0.0
    for i in range(B):
        ref = O.converse2d_op(x[i:i + 1], x0[i:i + 1], wt, b, s, 1e-5)
        err = max(err, float(np.abs(got[i:i + 1] - ref).max()))
    print(f"op planned B{B} C{C} {h}x{w} s{s} k{k} x0={x0kind}: max-abs {err:.3e}")
    assert err <= TOL


# (B, C, h, w, s, k, psf batch, act): module-level calls on the generic route with no padding and
# compile-time plans for h, w, h s and w s (the module column kernel k_modcols); the first is
# Converse-USRNet's first data step (converse_usrnet.py:205, 64^2 -> 256^2, per-sample 25 x 25 psf)
MODULE_PLANNED = [(4, 8, 64, 64, 4, 25, 4, None), (2, 3, 64, 128, 2, 5, 1, "gelu"), (1, 2, 128, 64, 3, 7, 1, None),
                  (2, 2, 256, 256, 2, 3, 2, None), (1, 2, 128, 192, 2, 4, 1, "gelu"), (1, 1, 256, 64, 4, 9, 1, None),
                  (1, 2, 64, 256, 3, 5, 1, None)]


@pytest.mark.parametrize("B,C,h,w,s,k,pb,act", MODULE_PLANNED)
def test_module_planned_scale(B, C, h, w, s, k, pb, act, monkeypatch):
    """Converse2D module path (util_converse.py:142-192) at scale > 1 without padding on the compile-time
    plans, against the fp64 oracle, max-abs <= 1e-4.  The generic route is forced (64 -> 256 at s = 4
    would otherwise take the fused upsampling kernel, tested in test_fused_upsampling_path)."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    lib = _lib.load()
    assert lib.cvn_converse2d_route(B, C, h, w, pb, k, k, s, 0) == _lib.ROUTE_GENERIC
    assert lib.cvn_converse2d_op_route(h, w, s) == _lib.ROUTE_OP_PLANNED  # the lengths have plans
    rng = seeded("module-planned", B, C, h, w, s, k, pb, act)
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    wt = (0.05 * rng.standard_normal((pb, C, k, k))).astype(np.float32) if pb > 1 else softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    dev = torch.device("cuda")
    got = Fh.converse2d_fused(torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev),
                              torch.from_numpy(b).to(dev).reshape(-1), s, 0, "circular", 1e-3, act,
                              cache=False).cpu().numpy()
    ref = O.converse2d_module(x, wt, b, s, 0, "circular", 1e-3)
    if act == "gelu":
        ref = O.gelu(ref)
    err = float(np.abs(got - ref).max())
    print(f"module planned B{B} C{C} {h}x{w} s{s} k{k} psf batch {pb} act {act}: max-abs {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("s,h,w", [(1, 30, 26), (4, 30, 26), (1, 32, 48), (2, 24, 20), (4, 16, 12)])
def test_op_level_large_psf(s, h, w):
    from conversenet_amd import functional as Fh
    rng = np.random.default_rng(77 + s + h)
    B, C, k = 2, 3, 25
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_op(x, x0, wt, b, s, 1e-5)
    dev = torch.device("cuda")
    got = Fh.converse2d_op(*(torch.from_numpy(a).to(dev) for a in (x, x0, wt, b)), s, 1e-5).cpu().numpy()
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("k", [2, 17, 34])
def test_table_split_dft_rows_psf_sizes(k):
    """Scale-1 tables on planes whose height is a multiple of 16 take the split-DFT evaluation of the
    transfer function (one to three psf rows per residue mod 16, even and odd sizes)."""
    rng = seeded("rows16", k)
    B, C, H, W = 1, 3, 64, 48
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k)
    b = (0.4 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_module(x, w, b, 1, 0, "circular", 1e-5)
    got = _run_fused(x, w, b, 1, 0, "circular", 1e-5)
    err = np.abs(got - ref).max()
    print(f"rows16 k{k}: max-abs {err:.3e}")
    assert err <= TOL, err


def test_module_biaseps_after_hip_forward():
    """The HIP path leaves biaseps = sigmoid(bias - 9) + eps readable after forward, as the reference's
    Converse2D.forward (util_converse.py:150) and ConvReverseDataNet.forward (converse_usrnet.py:46)."""
    from conversenet_amd.util_converse import Converse2D
    from conversenet_amd.converse_usrnet import ConvReverseDataNet
    dev = torch.device("cuda")
    m = Converse2D(4, 4, 3).to(dev)
    d = ConvReverseDataNet().to(dev)
    with torch.no_grad():
        m.bias.fill_(0.3)
        d.alpha.fill_(-0.2)
        m(torch.randn(1, 4, 12, 12, device=dev))
        d(torch.randn(1, 64, 8, 8, device=dev), torch.rand(1, 64, 3, 3, device=dev), 2)
    assert torch.allclose(m.biaseps, torch.sigmoid(m.bias - 9.0) + 1e-5)
    assert torch.allclose(d.biaseps, torch.sigmoid(d.alpha - 9.0) + 1e-3)


# ---------------------------------------------------------------------------------------------
# Fused upsampling path: HR plane 132 x 132 from LR planes of 66 (s = 2), 44 (s = 3), 33 (s = 4);
# HR plane 256 x 256 from LR planes of 64 (s = 4, Converse-USRNet's first data step)
# ---------------------------------------------------------------------------------------------
UP_CASES = [
    # (B, C, H, W, k, s, p, mode, psf batch)
    (2, 3, 64, 64, 3, 2, 1, "circular", 1),   # cfg2's geometry
    (1, 2, 62, 62, 5, 2, 2, "reflect", 1),
    (2, 2, 40, 40, 5, 3, 2, "replicate", 1),
    (1, 3, 31, 31, 4, 4, 1, "constant", 1),
    (2, 2, 33, 33, 7, 4, 0, "circular", 2),   # per-sample psf, no padding
    (2, 2, 64, 64, 25, 4, 0, "circular", 2),  # 256 plan: Converse-USRNet's data step (per-sample 25 x 25)
    (1, 3, 64, 64, 9, 4, 0, "replicate", 1),
    (1, 2, 62, 62, 5, 4, 1, "reflect", 1),    # 256 plan, padded LR plane, 248 x 248 output
    (2, 2, 60, 60, 4, 4, 2, "constant", 2),
    (2, 2, 64, 64, 61, 4, 0, "circular", 2),  # 256 plan, psf past the split-DFT table's LDS budget
]


@pytest.mark.parametrize("B,C,H,W,k,s,p,mode,pb", UP_CASES)
def test_fused_upsampling_path(B, C, H, W, k, s, p, mode, pb, monkeypatch):
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    rng = seeded("up", B, C, H, W, k, s, p, mode, pb)
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    w = softmax_psf(rng, C, k, pb)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    lib = _lib.load()
    assert lib.cvn_converse2d_route(B, C, H, W, pb, k, k, s, p) == _lib.ROUTE_FUSED
    dev = torch.device("cuda")
    xt, wt, bt = (torch.from_numpy(a).to(dev) for a in (x, w, b))
    got = Fh.converse2d_fused(xt, wt, bt.reshape(-1), s, p, mode, 1e-5).cpu().numpy()
    gelu = Fh.converse2d_fused(xt, wt, bt.reshape(-1), s, p, mode, 1e-5, act="gelu").cpu().numpy()
    ref = O.converse2d_module(x, w, b, s, p, mode, 1e-5)
    err = np.abs(got - ref).max()
    print(f"fused up B{B} C{C} {H}x{W} k{k} s{s} p{p} {mode} pb{pb}: max-abs {err:.3e}")
    assert err <= TOL
    assert np.abs(gelu - O.gelu(ref)).max() <= TOL
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    generic = Fh.converse2d_fused(xt, wt, bt.reshape(-1), s, p, mode, 1e-5).cpu().numpy()
    assert np.abs(generic - got).max() <= TOL
