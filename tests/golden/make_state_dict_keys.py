"""Writes tests/golden/state_dict_keys.json: parameter names and shapes of the reference's shipped
checkpoints (model_zoo/converse_dncnn.pth, converse_usrnet.pth, converse_srresnet.pth,
conversenet.pth), read with torch.load(weights_only=True).  Only names and shapes are kept (no
weights)."""
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ZOO = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/model_zoo"

out = {}
for name in ("converse_dncnn", "converse_usrnet", "converse_srresnet", "conversenet"):
    sd = torch.load(os.path.join(ZOO, name + ".pth"), map_location="cpu", weights_only=True)
    out[name] = {k: list(v.shape) for k, v in sd.items()}
with open(os.path.join(HERE, "state_dict_keys.json"), "w") as f:
    json.dump(out, f, indent=0, sort_keys=True)
print({k: len(v) for k, v in out.items()})
