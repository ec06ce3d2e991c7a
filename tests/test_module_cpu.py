"""Drop-in API of conversenet_amd.util_converse / converse_dncnn / converse_usrnet on the CPU:
constructor and backend behaviour of the reference (models/util_converse.py:99-169), state-dict
layout of the reference checkpoints, the registered converse2d op schema, and the PyTorch-backend
numerics (float64) against the oracle, including the full model compositions at small sizes."""
import json
import os

import numpy as np
import pytest
import torch

import conversenet_amd  # noqa: F401
from conversenet_amd import util_converse as U
from conversenet_amd.converse_dncnn import ConverseDnCNN
from conversenet_amd.converse_usrnet import ConverseUSRNet, ConvReverseDataNet
from oracle import converse_oracle as O
from tests.conftest import seeded

HERE = os.path.dirname(os.path.abspath(__file__))


def sd_numpy(m):
    return {k: v.detach().double().numpy() for k, v in m.state_dict().items()}


def test_converse2d_init_matches_reference_recipe():
    torch.manual_seed(0)
    m = U.Converse2D(4, 4, 5)
    torch.manual_seed(0)
    w = torch.softmax(torch.randn(1, 4, 5, 5).view(1, 4, -1), dim=-1).view(1, 4, 5, 5)
    torch.testing.assert_close(m.weight.data, w)
    assert torch.count_nonzero(m.bias) == 0 and m.bias.shape == (1, 4, 1, 1)
    assert set(m.state_dict()) == {"weight", "bias"}


def test_constructor_and_backend_errors():
    with pytest.raises(ValueError):
        U.Converse2D(2, 2, 3, backend="triton")
    with pytest.raises(AssertionError):
        U.Converse2D(2, 3, 3)
    m = U.Converse2D(2, 2, 3, padding=1, backend="cuda")
    with pytest.raises(RuntimeError, match="unavailable"):
        m(torch.randn(1, 2, 8, 8))


def test_env_backend_override(monkeypatch):
    m = U.Converse2D(2, 2, 3, padding=1)
    monkeypatch.setenv("CONVERSE2D_BACKEND", "cuda")
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 2, 8, 8))
    monkeypatch.setenv("CONVERSE2D_BACKEND", "pytorch")
    assert m(torch.randn(1, 2, 8, 8)).shape == (1, 2, 8, 8)


@pytest.mark.parametrize("mode", ["circular", "reflect", "replicate", "constant"])
@pytest.mark.parametrize("s", [1, 2, 3])
def test_pytorch_backend_float64_matches_oracle(mode, s):
    rng = seeded("mod", mode, s)
    m = U.Converse2D(3, 3, 4, scale=s, padding=2, padding_mode=mode).double()
    with torch.no_grad():
        m.bias.copy_(torch.from_numpy(0.3 * rng.standard_normal((1, 3, 1, 1))))
    x = rng.standard_normal((2, 3, 9, 11))
    y = m(torch.from_numpy(x)).detach().numpy()
    ref = O.converse2d_module(x, m.weight.detach().numpy(), m.bias.detach().numpy(), s, 2, mode, 1e-5)
    np.testing.assert_allclose(y, ref, atol=1e-9)
    assert torch.allclose(m.biaseps, torch.sigmoid(m.bias - 9.0) + 1e-5)


def test_registered_op_schema_and_cpu_semantics():
    op = torch.ops.converse2d.forward
    sch = op.default._schema
    assert [a.name for a in sch.arguments] == ["x", "x0", "weight", "bias", "scale", "eps"]
    assert [str(a.type) for a in sch.arguments] == ["Tensor"] * 4 + ["int", "float"]
    assert abs(sch.arguments[-1].default_value - 1e-5) < 1e-12
    rng = seeded("op")
    x, x0 = rng.standard_normal((1, 2, 8, 9)), rng.standard_normal((1, 2, 16, 18))
    w = rng.random((1, 2, 3, 3))
    b = rng.standard_normal((1, 2, 1, 1))
    got = op(*(torch.from_numpy(a) for a in (x, x0, w, b)), 2).numpy()
    np.testing.assert_allclose(got, O.converse2d_op(x, x0, w, b, 2, 1e-5), atol=1e-9)
    torch.ops.converse2d.clear_cache()
    with pytest.raises(RuntimeError, match="weight must be"):
        op(*(torch.from_numpy(a) for a in (x, x0, np.concatenate([w, w]), b)), 2)


def test_autograd_through_composite():
    torch.manual_seed(0)
    m = U.Converse2D(2, 2, 5, scale=2, padding=2).double()
    x = torch.randn(1, 2, 8, 9, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda t: m(t), (x,), eps=1e-6, atol=1e-4, rtol=1e-4)


def test_state_dict_layout_matches_reference_checkpoints():
    ref = json.load(open(os.path.join(HERE, "golden", "state_dict_keys.json")))
    mine = {k: list(v.shape) for k, v in ConverseDnCNN().state_dict().items()}
    assert mine == ref["converse_dncnn"]
    mine = {k: list(v.shape) for k, v in ConverseUSRNet().state_dict().items()}
    assert mine == ref["converse_usrnet"]
    assert sum(p.numel() for p in ConverseDnCNN().parameters()) == 796353


def test_converse_block_float64_matches_oracle():
    torch.manual_seed(1)
    blk = U.ConverseBlockAlphaVariant(8, 8, kernel_size=3, padding=2, padding_mode="circular").double()
    with torch.no_grad():
        blk.alpha1.normal_(0, 0.5)
        blk.alpha2.normal_(0, 0.5)
    x = torch.randn(2, 8, 12, 10, dtype=torch.float64)
    ref = O.converse_block(x.numpy(), sd_numpy(blk), "", 3, 1, 2, "circular", 1e-5, True)
    with torch.no_grad():
        np.testing.assert_allclose(blk(x).numpy(), ref, atol=1e-8)


def test_dncnn_float64_matches_oracle():
    torch.manual_seed(2)
    m = ConverseDnCNN().double().eval()
    x = torch.rand(1, 1, 12, 12, dtype=torch.float64)
    with torch.no_grad():
        y = m(x).numpy()
    np.testing.assert_allclose(y, O.converse_dncnn(x.numpy(), sd_numpy(m)), atol=1e-7)


def psnr(a, ref):
    """utils_image.py:626-641 with peak = dynamic range of the reference output."""
    mse = float(np.mean((a - ref) ** 2))
    return 10 * np.log10((ref.max() - ref.min()) ** 2 / mse) if mse > 0 else np.inf


def test_usrnet_matches_oracle():
    # KernelNet casts the kernel to float32 (converse_usrnet.py:134), so the model runs in fp32
    torch.manual_seed(3)
    m = ConverseUSRNet().eval()
    with torch.no_grad():
        for p in (m.d.alpha, *[b.alpha1 for b in m.p.m_body], *[b.alpha2 for b in m.p.m_body]):
            p.normal_(0, 0.1)
    x = torch.rand(1, 3, 6, 6)
    k = torch.rand(1, 1, 7, 7)
    k = k / k.sum()
    with torch.no_grad():
        y = m(x, k, 2).numpy()
    ref = O.converse_usrnet(x.numpy(), k.numpy(), 2, sd_numpy(m), 7)
    assert psnr(y, ref) > 60


def test_conv_reverse_datanet_per_sample_psf_matches_oracle():
    rng = seeded("crd")
    d = ConvReverseDataNet().double()
    with torch.no_grad():
        d.alpha.copy_(torch.from_numpy(rng.standard_normal((1, 64, 1, 1))))
    x = rng.standard_normal((2, 64, 6, 5))
    k = rng.random((2, 64, 3, 3))
    with torch.no_grad():
        y = d(torch.from_numpy(x), torch.from_numpy(k), 2).numpy()
    np.testing.assert_allclose(y, O.conv_reverse_datanet(x, k, 2, d.alpha.detach().numpy()), atol=1e-8)
