"""SRResNet family (conversenet_amd.converse_srresnet, models/converse_srresnet.py) on the CPU: the
plain layers of the oracle against torch, the three models against the oracle in fp64 on shared
state dicts, and the parameter layout against the reference's shipped checkpoints."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conversenet_amd.converse_srresnet import ConverseMSRResNet, ConverseUpMSRResNet
from conversenet_amd.converse_usrnet import ConverseNet
from oracle import converse_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
ZOO = "/root/reference/model_zoo"


def sd_numpy(m):
    return {k: v.detach().double().numpy() for k, v in m.state_dict().items()}


def test_plain_layers_match_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 3, 7, 9))
    w = rng.standard_normal((4, 3, 3, 3))
    b = rng.standard_normal(4)
    ref = F.conv2d(torch.tensor(x), torch.tensor(w), torch.tensor(b), padding=1).numpy()
    np.testing.assert_allclose(O.conv3x3(x, w, b), ref, atol=1e-12)
    for s in (2, 3, 4):
        ref = F.interpolate(torch.tensor(x), scale_factor=s, mode="bilinear", align_corners=False).numpy()
        np.testing.assert_allclose(O.bilinear_upsample(x, s), ref, atol=1e-12)


def test_converse_msrresnet_matches_oracle():
    torch.manual_seed(7)
    m = ConverseMSRResNet(num_features=16, num_blocks=1).double().eval()
    with torch.no_grad():
        for mod in (m.up1, m.up2):
            mod.bias.normal_(0, 0.5)
    x = torch.rand(1, 3, 6, 5, dtype=torch.float64)
    with torch.no_grad():
        y = m(x).numpy()
    np.testing.assert_allclose(y, O.converse_msrresnet(x.numpy(), sd_numpy(m), 1), atol=1e-8)


def test_converse_up_msrresnet_matches_oracle():
    torch.manual_seed(8)
    m = ConverseUpMSRResNet(num_features=16, num_blocks=2).double().eval()
    x = torch.rand(1, 3, 6, 6, dtype=torch.float64)
    with torch.no_grad():
        y = m(x).numpy()
    np.testing.assert_allclose(y, O.converse_up_msrresnet(x.numpy(), sd_numpy(m), 2), atol=1e-8)


def test_state_dict_layout_matches_reference_checkpoints():
    ref = json.load(open(os.path.join(HERE, "golden", "state_dict_keys.json")))
    assert {k: list(v.shape) for k, v in ConverseMSRResNet().state_dict().items()} == ref["converse_srresnet"]
    assert {k: list(v.shape) for k, v in ConverseNet().state_dict().items()} == ref["conversenet"]


@pytest.mark.skipif(not os.path.isdir(ZOO), reason="the reference's model_zoo is not on this machine")
def test_reference_checkpoint_loads_strict_and_runs():
    """The shipped ConverseMSRResNet weights (read with weights_only=True) load with strict=True and the
    model then agrees with the oracle evaluated on the same weights."""
    sd = torch.load(os.path.join(ZOO, "converse_srresnet.pth"), map_location="cpu", weights_only=True)
    m = ConverseMSRResNet()
    m.load_state_dict(sd, strict=True)
    m = m.double().eval()
    x = torch.rand(1, 3, 8, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        y = m(x).numpy()
    ref = O.converse_msrresnet(x.numpy(), sd_numpy(m))
    assert np.abs(y - ref).max() <= 1e-7 * max(1.0, np.abs(ref).max())
    ConverseNet().load_state_dict(torch.load(os.path.join(ZOO, "conversenet.pth"), map_location="cpu",
                                             weights_only=True), strict=True)
