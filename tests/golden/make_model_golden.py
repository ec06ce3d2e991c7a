"""Writes tests/golden/models_ref.npz: outputs of the reference's own model classes on small inputs.

Pins the compositions that no closed form covers: ConverseBlock and ConverseBlockAlphaVariant
(models/util_converse.py:253-323), ConverseDnCNN (models/converse_dncnn.py:11-35), ConvReverseDataNet
(models/converse_usrnet.py:33-117), KernelNet (:125-142), ConverseNet (:150-169), ConverseUSRNet
(:178-214) and ConverseMSRResNet / ConverseUpMSRResNet (models/converse_srresnet.py:50-119).

It imports those modules from the reference checkout, so it runs only in the build container, with
this repository kept off sys.path (the reference's extension probe, util_converse.py:10-34, must find
nothing and run its pure-PyTorch path) and without writing bytecode into the read-only checkout:
    python tests/golden/make_model_golden.py [/path/to/reference]

Parameter values are not stored: each case stores the (key, shape, kind) list of its state dict and a
seed, and tests/golden/model_params.py regenerates the values (see there).  Models run in float64
(`.double()`) except KernelNet and ConverseUSRNet, which cast their kernel input to float32
(converse_usrnet.py:134) and so run in float32.
"""
import json
import os
import sys

sys.dont_write_bytecode = True
HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:] = [p for p in sys.path if os.path.abspath(p or os.getcwd()) not in (REPO, os.path.dirname(HERE))]

import numpy as np  # noqa: E402
import torch  # noqa: E402
import torch.nn as nn  # noqa: E402

from model_params import seeded_state_dict  # noqa: E402  (sibling module in tests/golden)

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)

from models import util_converse as RU  # noqa: E402
from models import converse_dncnn as RD  # noqa: E402
from models import converse_usrnet as RN  # noqa: E402
from models import converse_srresnet as RS  # noqa: E402

assert not RU._HAS_CONVERSE2D_EXT, "an extension was found: run without this repository on sys.path"
OUT = os.path.join(HERE, "models_ref.npz")


def spec_of(model):
    """(key, shape, kind) for every parameter, in state-dict order."""
    kinds = {}
    for mname, mod in model.named_modules():
        for pname, _ in mod.named_parameters(recurse=False):
            key = f"{mname}.{pname}" if mname else pname
            if pname.startswith("alpha"):
                kind = "alpha"
            elif isinstance(mod, RU.Converse2D):
                kind = {"weight": "psf", "bias": "lam"}[pname]
            elif isinstance(mod, RU.LayerNorm):
                kind = {"weight": "ln_w", "bias": "ln_b"}[pname]
            elif isinstance(mod, (nn.Conv2d, nn.Linear)):
                kind = {"weight": "w", "bias": "b"}[pname]
            else:
                raise TypeError(f"unclassified parameter {key} of {type(mod).__name__}")
            kinds[key] = kind
    sd = model.state_dict()
    return [(k, list(v.shape), kinds[k]) for k, v in sd.items()]


def load_seeded(model, seed, dtype):
    spec = spec_of(model)
    vals = seeded_state_dict(spec, seed)
    model.load_state_dict({k: torch.from_numpy(v) for k, v in vals.items()}, strict=True)
    model.to(dtype).eval()
    return spec


def main():
    store = {}
    index = []

    def record(name, model, seed, dtype, inputs, run, **meta):
        spec = load_seeded(model, seed, dtype)
        with torch.no_grad():
            out = run(model, *[torch.from_numpy(a).to(dtype) if isinstance(a, np.ndarray) else a for a in inputs])
        store[f"{name}/spec"] = np.array(json.dumps(spec))
        store[f"{name}/seed"] = np.array(seed)
        store[f"{name}/meta"] = np.array(json.dumps(meta))
        for i, a in enumerate(inputs):
            if isinstance(a, np.ndarray):
                store[f"{name}/in{i}"] = a
        store[f"{name}/out"] = out.numpy()
        index.append(name)
        print(f"{name}: out {tuple(out.shape)} {out.dtype} range [{out.min():.4g}, {out.max():.4g}]")

    rng = np.random.default_rng(20251202)
    f64 = torch.float64

    # ConverseBlock / ConverseBlockAlphaVariant: (kernel, padding, mode, alpha variant, B, C, H, W)
    for i, (k, p, mode, alpha, B, C, H, W) in enumerate([(3, 2, "circular", False, 2, 4, 10, 12),
                                                         (5, 2, "replicate", True, 1, 4, 9, 11),
                                                         (7, 6, "circular", True, 1, 4, 12, 10),
                                                         (3, 1, "reflect", False, 1, 4, 8, 8),
                                                         (4, 2, "circular", True, 1, 4, 10, 10)]):
        cls = RU.ConverseBlockAlphaVariant if alpha else RU.ConverseBlock
        x = rng.standard_normal((B, C, H, W))
        record(f"block{i}", cls(C, C, kernel_size=k, scale=1, padding=p, padding_mode=mode), 100 + i, f64, [x],
               lambda m, x: m(x), kernel_size=k, padding=p, padding_mode=mode, alpha=alpha)

    # ConverseDnCNN(): default k7 p6 circular, 20 blocks
    x = 0.5 + 0.3 * rng.standard_normal((1, 1, 20, 20))
    record("dncnn", RD.ConverseDnCNN(), 200, f64, [x], lambda m, x: m(x))

    # ConvReverseDataNet with a per-sample psf: (sf, B, H, W, kernel, padding, mode)
    for i, (sf, B, H, W, k, p, mode) in enumerate([(1, 2, 6, 7, 5, 0, "circular"), (2, 2, 5, 5, 5, 0, "circular"),
                                                   (4, 1, 4, 4, 7, 0, "circular"), (2, 1, 5, 6, 3, 2, "reflect")]):
        x = rng.standard_normal((B, 64, H, W))
        kk = 0.2 * rng.standard_normal((B, 64, k, k))
        record(f"datanet{i}", RN.ConvReverseDataNet(), 300 + i, f64, [x, kk, sf, p, mode],
               lambda m, x, kk, sf, p, mode: m(x, kk, sf, padding=p, padding_mode=mode), sf=sf, padding=p,
               padding_mode=mode)

    # KernelNet(7) (float32: its forward casts the kernel to float)
    kk = rng.random((2, 1, 7, 7)).astype(np.float32)
    kk /= kk.sum(axis=(2, 3), keepdims=True)
    record("kernelnet", RN.KernelNet(), 400, torch.float32, [kk], lambda m, k: m(k))

    # ConverseNet (MultiConverseBlock, repeated iterations), float64
    x = rng.random((1, 3, 8, 8))
    record("conversenet", RN.ConverseNet(num_iterations=2, num_blocks=2), 500, f64, [x], lambda m, x: m(x),
           num_iterations=2, num_blocks=2)

    # ConverseUSRNet (float32): 7x7 blur kernels (KernelNet() is 7x7), sf on the first iteration only
    for i, (sf, H) in enumerate([(2, 8), (3, 6)]):
        x = rng.random((1, 3, H, H)).astype(np.float32)
        kk = rng.random((1, 1, 7, 7)).astype(np.float32)
        kk /= kk.sum()
        record(f"usrnet{i}", RN.ConverseUSRNet(), 600 + i, torch.float32, [x, kk, sf],
               lambda m, x, k, sf: m(x, k, sf), sf=sf)

    # SRResNet family with two body blocks, x4
    x = rng.random((1, 3, 6, 6))
    record("converse_msrresnet", RS.ConverseMSRResNet(num_blocks=2), 700, f64, [x], lambda m, x: m(x), num_blocks=2)
    record("converse_up_msrresnet", RS.ConverseUpMSRResNet(num_blocks=2), 701, f64, [x], lambda m, x: m(x),
           num_blocks=2)

    store["index"] = np.array(json.dumps(index))
    np.savez_compressed(OUT, **store)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
