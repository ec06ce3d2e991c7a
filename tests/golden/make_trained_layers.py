"""Writes tests/golden/trained_layers.npz: the psf (`conv1.3.weight`) and bias (`conv1.3.bias`) of the
trained Converse2D layer with the smallest regularisation weight lambda = sigmoid(bias - 9) + eps in
each of the reference's shipped checkpoints that has one (model_zoo/converse_dncnn.pth,
converse_usrnet.pth, converse_srresnet.pth), plus Converse-USRNet's data-step `d.alpha`.  Read with
torch.load(weights_only=True); only these few arrays are kept (about 45 KB).

Trained biases reach -1.83 (Converse-USRNet body block 3), so lambda falls to 3.0e-5 against 1.33e-4
at the default initialisation, and the solve's largest spectral gain 1 / (2 sqrt(lambda)) rises from
43 to 91: the GPU tests run these layers at the models' own layer shapes against the fp64 oracle."""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ZOO = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/model_zoo"
EPS = 1e-5  # Converse2D's default eps (models/util_converse.py:99), used by every body block

out = {}
for name in ("converse_dncnn", "converse_usrnet", "converse_srresnet"):
    sd = torch.load(os.path.join(ZOO, name + ".pth"), map_location="cpu", weights_only=True)
    layers = [k[:-len(".bias")] for k, v in sd.items() if k.endswith("conv1.3.bias") and v.dim() == 4]
    lam = {k: float((torch.sigmoid(sd[k + ".bias"].double() - 9) + EPS).min()) for k in layers}
    k = min(lam, key=lam.get)
    out[f"{name}.layer"] = np.array(k)
    out[f"{name}.weight"] = sd[k + ".weight"].float().numpy()
    out[f"{name}.bias"] = sd[k + ".bias"].float().numpy()
    out[f"{name}.lambda_min"] = np.array(lam[k])
    if name == "converse_usrnet":
        out["converse_usrnet.d.alpha"] = sd["d.alpha"].float().numpy()
    print(name, k, tuple(sd[k + ".weight"].shape), f"lambda_min {lam[k]:.3e}")
np.savez_compressed(os.path.join(HERE, "trained_layers.npz"), **out)
