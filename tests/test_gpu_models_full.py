"""Full-size model and pointwise parity on the GPU against the fp64 oracle.

cfg4: Converse-DnCNN (models/converse_dncnn.py:11-35, default k7 p6, 20 blocks) on one 1x256x256 image
of the benchmark's synthetic batch: every Converse2D runs the 268 x 268 path (row pass, column pass,
inverse row pass) and the chained block tail with the next block's head.
cfg5: Converse-USRNet (models/converse_usrnet.py:178-214) with KernelNet(25), non-zero alphas, one
3x64x64 LR image of the benchmark's batch blurred by its 25x25 kernel, x4: the data step at s = 4 with a
per-sample 25x25 psf (64 -> 256), then 260 x 260 body blocks on the fused kernel.
Gate (north star): PSNR >= 60 dB against the oracle, peak = dynamic range of the oracle output.
cfg3 LayerNorm / 1x1+GELU: the benchmark's own shape (B16 C64 256x256), max-abs <= 1e-4.
"""
import numpy as np
import pytest
import torch

import bench
from oracle import converse_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _sd(m):
    return {k: v.detach().cpu().numpy() for k, v in m.state_dict().items()}


def psnr(a, ref):
    mse = float(np.mean((a.astype(np.float64) - ref) ** 2))
    return 10 * np.log10((ref.max() - ref.min()) ** 2 / mse) if mse > 0 else np.inf


def test_converse_dncnn_cfg4_full_size():
    from conversenet_amd import functional as Fh
    m, x = bench.make_dncnn(torch, DEV, batch=1)
    assert sum(p.numel() for p in m.parameters()) == 796353
    h0 = Fh.table_cache.misses
    with torch.no_grad():
        got = m(x).cpu().numpy()
    assert Fh.table_cache.misses - h0 == 20  # one 268-route table per block
    assert all(k[7] == 2 for k in list(Fh.table_cache.entries)[-20:])  # CVN_ROUTE_PFA268
    ref = O.converse_dncnn(x.cpu().numpy(), _sd(m))
    p = psnr(got, ref)
    print(f"cfg4 Converse-DnCNN 1x256x256: PSNR {p:.1f} dB, max-abs {np.abs(got - ref).max():.3e}, "
          f"|ref| max {np.abs(ref).max():.3f}")
    assert p >= 60


def test_converse_usrnet_cfg5_full_size():
    m, x, k = bench.make_usrnet(torch, DEV, batch=1)
    assert m.kernelnet.kernel_size == 25 and tuple(k.shape) == (1, 1, 25, 25)
    sd = _sd(m)
    assert np.abs(sd["d.alpha"]).max() > 0 and np.abs(sd["p.m_body.0.alpha1"]).max() > 0
    with torch.no_grad():
        got = m(x, k, 4).cpu().numpy()
    assert got.shape == (1, 3, 256, 256)
    ref = O.converse_usrnet(x.cpu().numpy(), k.cpu().numpy(), 4, sd, 25)
    p = psnr(got, ref)
    print(f"cfg5 Converse-USRNet 1x3x64x64 -> 256x256: PSNR {p:.1f} dB, max-abs {np.abs(got - ref).max():.3e}, "
          f"|ref| max {np.abs(ref).max():.3f}")
    assert p >= 60


@pytest.mark.parametrize("what", ["layernorm", "conv1x1_gelu"])
def test_cfg3_pointwise_full_shape(what):
    """The benchmark's LayerNorm (eps 1e-6) and 1x1 64->64 + GELU at B16 C64 256x256 against the oracle
    over every pixel (the oracle runs one batch element at a time to bound host memory)."""
    from conversenet_amd import functional as Fh
    x, _, _ = bench.make_cfg3_inputs(torch)
    xd = x.to(DEV)
    if what == "layernorm":
        g = torch.Generator().manual_seed(5)
        lw, lb = 1 + 0.1 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g)
        got = Fh.layernorm_cf(xd, lw.to(DEV), lb.to(DEV), 1e-6).cpu().numpy()
        ref = lambda xb: O.layernorm_cf(xb, lw.numpy(), lb.numpy(), 1e-6)  # noqa: E731
    else:
        torch.manual_seed(2)
        conv = torch.nn.Conv2d(64, 64, 1)
        got = Fh.conv1x1(xd, conv.weight.to(DEV), conv.bias.to(DEV), act="gelu").cpu().numpy()
        wn, bn = conv.weight.detach().numpy(), conv.bias.detach().numpy()
        ref = lambda xb: O.gelu(O.conv1x1(xb, wn, bn))  # noqa: E731
    xn = x.numpy()
    err = max(float(np.abs(got[b:b + 1] - ref(xn[b:b + 1])).max()) for b in range(xn.shape[0]))
    print(f"cfg3 {what} B16 C64 256x256: max-abs {err:.3e}")
    assert err <= 1e-4
