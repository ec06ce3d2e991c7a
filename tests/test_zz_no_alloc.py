"""cvn_converse2d_fwd_noalloc_f32 (the allocation-free forward, scratch in a file-scope device array)
against cvn_converse2d_fwd_f32 (caller workspace) through the C ABI: two calls in a row on each route,
the second with a smaller input, so the second call runs over the first call's leftovers in the array.
Both run the same kernels, so the outputs must be identical."""
import numpy as np
import pytest
import torch

from conversenet_amd import _lib
from oracle import converse_oracle as O
from tests.conftest import seeded, softmax_psf

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

# (B, C, H, W, k, s, pad, mode) pairs: larger first, smaller second
PAIRS = {
    "fused": [(4, 64, 256, 256, 5, 1, 2, "circular"), (1, 8, 128, 128, 5, 1, 2, "reflect")],
    "generic": [(2, 16, 64, 64, 3, 1, 1, "circular"), (2, 3, 30, 26, 5, 3, 2, "replicate")],
    "pfa268": [(2, 8, 256, 256, 7, 1, 6, "circular"), (1, 2, 256, 256, 5, 1, 6, "constant")],
}
ROUTE_IDS = {"fused": _lib.ROUTE_FUSED, "generic": _lib.ROUTE_GENERIC, "pfa268": _lib.ROUTE_PFA268}


def _inputs(B, C, H, W, k, s, p, mode):
    rng = seeded("noalloc", B, C, H, W, k, s, p, mode)
    x = torch.from_numpy(rng.standard_normal((B, C, H, W)).astype(np.float32)).to(DEV)
    w = torch.from_numpy(softmax_psf(rng, C, k)).to(DEV)
    b = torch.from_numpy((0.3 * rng.standard_normal(C)).astype(np.float32)).to(DEV)
    return x, w, b


def _both(lib, x, w, b, s, p, mode, act):
    B, C, H, W = x.shape
    k = w.shape[-1]
    st = torch.cuda.current_stream().cuda_stream
    args = (x.data_ptr(), B, C, H, W, w.data_ptr(), 1, k, k, b.data_ptr(), 1e-5, s, p, _lib.PAD_MODES[mode], act)
    nb = lib.cvn_converse2d_fwd_workspace(B, C, H, W, 1, k, k, s, p)
    assert 0 < nb <= _lib.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    ref = torch.empty((B, C, H * s, W * s), device=DEV)
    got = torch.full_like(ref, float("nan"))
    _lib.check(lib.cvn_converse2d_fwd_f32(*args, ref.data_ptr(), ws.data_ptr(), nb, st), "fwd")
    _lib.check(lib.cvn_converse2d_fwd_noalloc_f32(*args, got.data_ptr(), st), "fwd_noalloc")
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("route", list(PAIRS))
def test_noalloc_matches_workspace_entry_point(route):
    lib = _lib.load()
    for i, (B, C, H, W, k, s, p, mode) in enumerate(PAIRS[route]):
        print(f"noalloc {route} call {i}: B{B} C{C} {H}x{W} k{k} s{s} p{p} {mode}", flush=True)
        assert lib.cvn_converse2d_route(B, C, H, W, 1, k, k, s, p) == ROUTE_IDS[route]
        x, w, b = _inputs(B, C, H, W, k, s, p, mode)
        act = _lib.ACT_GELU if i == 1 else _lib.ACT_NONE
        ref, got = _both(lib, x, w, b, s, p, mode, act)
        assert torch.equal(ref, got), float((ref - got).abs().max())
        if i == 1:  # the smaller call also against the oracle
            o = O.gelu(O.converse2d_module(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy().reshape(1, C, 1, 1), s,
                                           p, mode, 1e-5))
            assert np.abs(got.cpu().numpy() - o).max() <= 1e-4


def test_noalloc_rejects_calls_above_its_scratch():
    lib = _lib.load()
    B, C, H, W, k, s, p = 8, 128, 256, 256, 7, 1, 6  # a Converse-DnCNN layer: ~330 MB of workspace
    assert lib.cvn_converse2d_fwd_workspace(B, C, H, W, 1, k, k, s, p) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.empty(1, device=DEV)
    rc = lib.cvn_converse2d_fwd_noalloc_f32(x.data_ptr(), B, C, H, W, x.data_ptr(), 1, k, k, x.data_ptr(), 1e-5, s, p,
                                            3, 0, x.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.CVN_ERR_UNSUPPORTED and b"scratch" in lib.cvn_last_error()
