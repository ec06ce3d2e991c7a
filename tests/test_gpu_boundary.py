"""The drop-in boundary on the GPU: the registered op torch.ops.converse2d.forward with data (its HIP
dispatch and cached op table), the one-shot C entry point, explicit routes and cached tables across an
environment change, inference mode, the cache staying bounded, and geometries outside the library's
limits running the composition instead of raising."""
import numpy as np
import pytest
import torch

from oracle import converse_oracle as O
from tests.conftest import seeded, softmax_psf

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
TOL = 1e-4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("s", [1, 2])
def test_registered_op_with_data(s):
    """torch.ops.converse2d.forward (converse2d.cpp:218-227 schema) on HIP tensors runs the library
    (op table cached on the first call, hit on the second) and matches the reference op's arithmetic."""
    import conversenet_amd  # noqa: F401  (registers the namespace)
    from conversenet_amd import functional as Fh
    rng = seeded("op", s)
    B, C, h, w, k = 2, 5, 36, 30, 5
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    x0 = rng.standard_normal((B, C, h * s, w * s)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    ref = O.converse2d_op(x, x0, wt, b, s, 1e-5)
    xt, x0t, wtt, bt = (_t(a) for a in (x, x0, wt, b))
    hits, misses = Fh.table_cache.hits, Fh.table_cache.misses
    with torch.no_grad():
        got1 = torch.ops.converse2d.forward(xt, x0t, wtt, bt, s, 1e-5).cpu().numpy()
        got2 = torch.ops.converse2d.forward(xt, x0t, wtt, bt, s, 1e-5).cpu().numpy()
    assert Fh.table_cache.misses == misses + 1 and Fh.table_cache.hits == hits + 1
    err = max(np.abs(got1 - ref).max(), np.abs(got2 - ref).max())
    print(f"converse2d::forward s={s}: max-abs {err:.3e}")
    assert err <= TOL
    # a new psf value in place: the cached table must not be reused
    with torch.no_grad():
        wtt.mul_(0.5).add_(0.5 / (k * k))
        got3 = torch.ops.converse2d.forward(xt, x0t, wtt, bt, s, 1e-5).cpu().numpy()
    ref3 = O.converse2d_op(x, x0, 0.5 * wt + 0.5 / (k * k), b, s, 1e-5)
    assert np.abs(got3 - ref3).max() <= TOL
    # clear_cache drops the tables (converse2d.cpp:211-216)
    torch.ops.converse2d.clear_cache()
    assert Fh.table_cache.bytes == 0


@pytest.mark.parametrize("h,w", [(36, 30), (260, 260)])
def test_registered_op_x0_is_x(h, w):
    """The reference module's scale-1 call passes x0 = x (util_converse.py:166): the op then takes the
    module route on the padded plane; the result is the op's, for an x whose border is arbitrary."""
    rng = seeded("op-alias", h, w)
    B, C, k = 2, 3, 5
    x = rng.standard_normal((B, C, h, w)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    xt = _t(x)
    with torch.no_grad():
        got = torch.ops.converse2d.forward(xt, xt, _t(wt), _t(b), 1, 1e-5).cpu().numpy()
    ref = O.converse2d_op(x, x, wt, b, 1, 1e-5)
    err = np.abs(got - ref).max()
    print(f"converse2d::forward x0 is x {h}x{w}: max-abs {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("H,k,p,s", [(256, 5, 2, 1), (256, 7, 6, 1), (40, 3, 1, 2), (30, 5, 2, 3)])
def test_one_shot_entry_point(H, k, p, s):
    """cvn_converse2d_fwd_f32 with data on each route: fused 260^2, 268 path, generic s = 2 / 3."""
    from conversenet_amd import functional as Fh
    rng = seeded("oneshot", H, k, p, s)
    B, C = 2, 3
    x = rng.standard_normal((B, C, H, H)).astype(np.float32)
    wt = softmax_psf(rng, C, k)
    b = (0.3 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
    got = Fh.converse2d_fwd_oneshot(_t(x), _t(wt), _t(b).reshape(-1), s, p, "circular", 1e-5).cpu().numpy()
    ref = O.converse2d_module(x, wt, b, s, p, "circular", 1e-5)
    err = np.abs(got - ref).max()
    print(f"one-shot {H}^2 k{k} p{p} s{s}: max-abs {err:.3e}")
    assert err <= TOL


def test_cached_table_survives_environment_change(monkeypatch):
    """A table cached on the fused route stays correct after CVN_DISABLE_FUSED=1 selects the generic
    route for new tables: the route is part of the cache key and travels with the table."""
    from conversenet_amd import _lib
    from conversenet_amd import functional as Fh
    rng = seeded("route-env")
    B, C, H = 2, 4, 256
    x = _t(rng.standard_normal((B, C, H, H)).astype(np.float32))
    wt = _t(softmax_psf(rng, C, 5))
    b = torch.zeros(C, device=DEV)
    monkeypatch.delenv("CVN_DISABLE_FUSED", raising=False)
    y_fused = Fh.converse2d_fused(x, wt, b, 1, 2, "circular", 1e-5)
    assert list(Fh.table_cache.entries)[-1][7] == _lib.ROUTE_FUSED
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    y_gen = Fh.converse2d_fused(x, wt, b, 1, 2, "circular", 1e-5)
    assert list(Fh.table_cache.entries)[-1][7] == _lib.ROUTE_GENERIC
    monkeypatch.delenv("CVN_DISABLE_FUSED")
    y_again = Fh.converse2d_fused(x, wt, b, 1, 2, "circular", 1e-5)  # cached fused table, fused route
    ref = O.converse2d_module(x.cpu().numpy(), wt.cpu().numpy(), np.zeros((1, C, 1, 1), np.float32), 1, 2,
                              "circular", 1e-5)
    for y in (y_fused, y_gen, y_again):
        assert np.abs(y.cpu().numpy() - ref).max() <= TOL


def test_inference_mode_models_and_cache_bound():
    """Converse2D and Converse-USRNet under torch.inference_mode (the per-sample psf is then an inference
    tensor without a version counter), and the table cache staying flat over repeated forwards."""
    from conversenet_amd import functional as Fh
    from conversenet_amd.converse_usrnet import ConverseUSRNet
    from conversenet_amd.util_converse import Converse2D
    torch.manual_seed(3)
    m = ConverseUSRNet().to(DEV).eval()
    with torch.no_grad():
        for prm in (m.d.alpha, *[blk.alpha1 for blk in m.p.m_body], *[blk.alpha2 for blk in m.p.m_body]):
            prm.normal_(0, 0.1)
    cv = Converse2D(8, 8, 3, scale=2, padding=1).to(DEV)
    rng = seeded("infer")
    x = _t(rng.random((1, 3, 12, 12)).astype(np.float32))
    k = rng.random((1, 1, 7, 7)).astype(np.float32)
    k = _t(k / k.sum())
    xc = torch.randn(2, 8, 10, 12, device=DEV)
    with torch.no_grad():
        ref_m = m(x, k, 2).cpu().numpy()
        ref_c = cv(xc).cpu().numpy()
    sizes = []
    with torch.inference_mode():
        for _ in range(3):
            got_m = m(x, k, 2).cpu().numpy()
            got_c = cv(xc).cpu().numpy()
            sizes.append((len(Fh.table_cache.entries), Fh.table_cache.bytes))
    assert np.abs(got_m - ref_m).max() <= 1e-4 * max(1.0, np.abs(ref_m).max())
    assert np.abs(got_c - ref_c).max() <= 1e-6
    assert sizes[0] == sizes[1] == sizes[2], sizes
    print("cache entries / bytes over inference forwards:", sizes)


def test_training_steps_leave_no_dead_tables():
    """Training through Converse2D (library forward and backward) with optimizer steps: the table cache
    does not grow, and an eval forward after the steps sees the updated weights."""
    from conversenet_amd import functional as Fh
    from conversenet_amd.util_converse import Converse2D
    torch.manual_seed(4)
    m = Converse2D(4, 4, 5, padding=2).to(DEV)
    opt = torch.optim.SGD(m.parameters(), lr=1e-3)
    x = torch.randn(2, 4, 24, 20, device=DEV)
    n0, b0 = len(Fh.table_cache.entries), Fh.table_cache.bytes
    for _ in range(4):
        opt.zero_grad()
        m(x).square().mean().backward()
        opt.step()
        with torch.no_grad():
            m(x)
    assert len(Fh.table_cache.entries) <= n0 + 1 and Fh.table_cache.bytes <= b0 + 4 * 4096 * 1024
    with torch.no_grad():
        got = m(x).cpu().numpy()
    ref = O.converse2d_module(x.cpu().numpy(), m.weight.detach().cpu().numpy(), m.bias.detach().cpu().numpy(), 1, 2,
                              "circular", 1e-5)
    assert np.abs(got - ref).max() <= TOL


def test_outside_library_limits_runs_the_composition():
    """A padded side above 4096 and weight gradients at scale 5 are outside the library's limits: the
    module runs the PyTorch composition (torch.fft on the GPU) instead of raising."""
    from conversenet_amd.util_converse import Converse2D
    torch.manual_seed(5)
    m = Converse2D(1, 1, 3, padding=1).to(DEV)
    x = torch.randn(1, 1, 4100, 6, device=DEV)
    with torch.no_grad():
        got = m(x).cpu().numpy()
    ref = O.converse2d_module(x.cpu().numpy(), m.weight.detach().cpu().numpy(), m.bias.detach().cpu().numpy(), 1, 1,
                              "circular", 1e-5)
    err = np.abs(got - ref).max()
    print(f"4100x6 plane on the composition: max-abs {err:.3e}")
    # the composition keeps the reference's fp32 op order, whose (FR - FBC invWBR) / lambda cancellation
    # costs up to a few 1e-3 against the exact (fp64) result
    assert err <= 1e-2
    up = Converse2D(2, 2, 3, scale=5, padding=1).to(DEV)
    xs = torch.randn(1, 2, 6, 7, device=DEV)
    up(xs).sum().backward()  # weight gradients at s = 5: composition under autograd
    assert up.weight.grad is not None and torch.isfinite(up.weight.grad).all()


def test_registered_ops_outside_library_limits_run_the_composition():
    """converse2d::forward and converse2d::forward_fused on HIP tensors whose geometry the library does
    not serve (a padded side above 4096) run the PyTorch composition instead of raising
    CVN_ERR_UNSUPPORTED (the reference op has no such limits, converse2d.cpp:165-209)."""
    import conversenet_amd  # noqa: F401  (registers torch.ops.converse2d)
    torch.manual_seed(6)
    w = torch.softmax(torch.randn(1, 1, 9), -1).reshape(1, 1, 3, 3).to(DEV)
    b = torch.zeros(1, 1, 1, 1, device=DEV)
    xp = torch.randn(1, 1, 4100, 6, device=DEV)  # already padded, as the op takes it
    x0 = torch.randn(1, 1, 4100, 6, device=DEV)
    with torch.no_grad():
        got = torch.ops.converse2d.forward(xp, x0, w, b, 1, 1e-5).cpu().numpy()
        fused = torch.ops.converse2d.forward_fused(xp[..., 1:-1, 1:-1].contiguous(), w, b, 1, 1, "circular",
                                                   1e-5).cpu().numpy()
    ref = O.converse2d_op(xp.cpu().numpy(), x0.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy(), 1, 1e-5)
    ref_f = O.converse2d_module(xp[..., 1:-1, 1:-1].cpu().numpy(), w.cpu().numpy(), b.cpu().numpy(), 1, 1,
                                "circular", 1e-5)
    err, err_f = np.abs(got - ref).max(), np.abs(fused - ref_f).max()
    print(f"op 4100x6 on the composition: max-abs {err:.3e}; forward_fused {err_f:.3e}")
    assert got.shape == (1, 1, 4100, 6) and fused.shape == (1, 1, 4098, 4)
    assert err <= 1e-2 and err_f <= 1e-2  # the reference's fp32 op order (see above)


def test_pfa268_route_rejects_misaligned_table():
    """The 268 path copies table entries with 16-byte direct-to-LDS loads: an apply on
    CVN_ROUTE_PFA268 with a table that is not 16-byte aligned returns CVN_ERR_ARG before any launch,
    and the same table aligned runs and matches the oracle."""
    from conversenet_amd import _lib
    lib = _lib.load()
    rng = seeded("pfa268-align")
    B, C, H, k, p = 1, 2, 256, 7, 6
    x = _t(rng.standard_normal((B, C, H, H)).astype(np.float32))
    wt = softmax_psf(rng, C, k)
    b = np.zeros((1, C, 1, 1), np.float32)
    wtt, bt = _t(wt), _t(b.reshape(-1))
    assert lib.cvn_converse2d_route(B, C, H, H, 1, k, k, 1, p) == _lib.ROUTE_PFA268
    tb = lib.cvn_converse2d_table_bytes(B, C, H, H, 1, k, k, 1, p, _lib.ROUTE_PFA268)
    sb = lib.cvn_converse2d_scratch_bytes(B, C, H, H, 1, k, k, 1, p, _lib.ROUTE_PFA268)
    table = torch.empty(tb + 16, dtype=torch.uint8, device=DEV)
    scratch = torch.empty(sb, dtype=torch.uint8, device=DEV)
    out = torch.empty((B, C, H, H), dtype=torch.float32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.cvn_converse2d_table_f32(wtt.data_ptr(), 1, k, k, bt.data_ptr(), 1e-5, B, C, H, H, 1, p,
                                        _lib.ROUTE_PFA268, table.data_ptr(), tb, st) == _lib.CVN_OK
    args = (x.data_ptr(), B, C, H, H, 1, k, k, 1, p, _lib.PAD_MODES["circular"], 0, _lib.ROUTE_PFA268)
    rc = lib.cvn_converse2d_apply_f32(*args, table.data_ptr() + 8, tb, scratch.data_ptr(), sb, out.data_ptr(), st)
    assert rc == _lib.CVN_ERR_ARG
    rc = lib.cvn_converse2d_apply_f32(*args, table.data_ptr(), tb, scratch.data_ptr(), sb, out.data_ptr(), st)
    assert rc == _lib.CVN_OK
    torch.cuda.synchronize()
    ref = O.converse2d_module(x.cpu().numpy(), wt, b, 1, p, "circular", 1e-5)
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL


def test_backward_with_misaligned_workspace():
    """The backward lays its workspace regions out from a 256-byte boundary inside the caller's buffer
    (its kernels use 16-byte loads and direct-to-LDS copies): a workspace pointer 8 bytes past an
    aligned one, with the queried size, gives the aligned call's gradients."""
    from conversenet_amd import _lib
    lib = _lib.load()
    rng = seeded("bwd-align")
    B, C, H, k, p = 2, 2, 256, 5, 2
    x = _t(rng.standard_normal((B, C, H, H)).astype(np.float32))
    g = _t(rng.standard_normal((B, C, H, H)).astype(np.float32))
    wt = _t(softmax_psf(rng, C, k))
    b = _t((0.3 * rng.standard_normal(C)).astype(np.float32))
    nb = lib.cvn_converse2d_bwd_workspace(B, C, H, H, 1, k, k, 1, p)
    ws = torch.empty(nb + 64, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    res = []
    for off in (0, 8):
        gx = torch.empty_like(x)
        gw = torch.empty((1, C, k, k), dtype=torch.float32, device=DEV)
        gb = torch.empty(C, dtype=torch.float32, device=DEV)
        rc = lib.cvn_converse2d_bwd_f32(g.data_ptr(), x.data_ptr(), B, C, H, H, wt.data_ptr(), 1, k, k,
                                        b.data_ptr(), 1e-5, 1, p, _lib.PAD_MODES["circular"], gx.data_ptr(),
                                        gw.data_ptr(), gb.data_ptr(), ws.data_ptr() + off, nb, st)
        assert rc == _lib.CVN_OK
        torch.cuda.synchronize()
        res.append((gx.cpu().numpy(), gw.cpu().numpy(), gb.cpu().numpy()))
    for a0, a1 in zip(*res):
        assert np.abs(a0 - a1).max() <= 1e-5 * max(1.0, np.abs(a0).max())
