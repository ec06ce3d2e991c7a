"""Writes tests/golden/converse2d_ref.npz: input/output vectors of the reference's own Converse2D op.

The outputs come from the reference C++ op (Converse2D/torch_converse2d/converse2d.cpp) compiled
from its source by oracle/Makefile into oracle/_ref/converse2d_ref.so, run on the CPU in float64 and
float32.  Module-level cases wrap the op exactly as Converse2D.forward does
(models/util_converse.py:144-190): F.pad, x0 = x (s == 1) or nearest upsample, op, crop.
Per-sample psf cases (ConvReverseDataNet, models/converse_usrnet.py:77-104) run the op once per
sample with that sample's psf, which is the same arithmetic.

Run in a process that has not imported conversenet_amd (both define the converse2d op namespace):
    python tests/golden/make_golden.py
"""
import itertools
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.path.join(ROOT, "oracle", "_ref", "converse2d_ref.so")


def softmax_psf(rng, batch, C, k):
    w = rng.standard_normal((batch, C, k * k))
    w = np.exp(w - w.max(-1, keepdims=True))
    return (w / w.sum(-1, keepdims=True)).reshape(batch, C, k, k).astype(np.float32)


def module_forward(x, w, b, s, p, mode, eps, dtype):
    x, w, b = (torch.from_numpy(a).to(dtype) for a in (x, w, b))
    y = F.pad(x, [p] * 4, mode=mode, value=0) if p > 0 else x
    x0 = y if s == 1 else F.interpolate(y, scale_factor=s, mode="nearest")
    outs = []
    for i in range(w.shape[0]):  # psf batch 1 (shared) or B (per sample)
        yi = y if w.shape[0] == 1 else y[i:i + 1]
        x0i = x0 if w.shape[0] == 1 else x0[i:i + 1]
        outs.append(torch.ops.converse2d.forward(yi, x0i, w[i:i + 1], b, s, eps))
    out = torch.cat(outs, 0) if len(outs) > 1 else outs[0]
    if p > 0:
        out = out[..., p * s:-p * s, p * s:-p * s]
    return out.numpy()


def main():
    torch.ops.load_library(REF)
    rng = np.random.default_rng(20240601)
    cases = []
    # (B, C, H, W, k, s, p, mode, psf_batch, eps)
    for (H, W), k, s in itertools.product([(16, 18), (9, 14)], [3, 5], [1, 2]):
        cases.append((1, 2, H, W, k, s, k // 2, "circular", 1, 1e-5))
    for mode, s in itertools.product(["reflect", "replicate", "constant", "circular"], [1, 2, 3]):
        cases.append((1, 2, 9, 11, 4, s, 3, mode, 1, 1e-5))
    cases.append((1, 2, 7, 9, 3, 4, 1, "reflect", 1, 1e-5))
    cases.append((1, 3, 12, 12, 2, 2, 1, "replicate", 1, 1e-3))  # SRResNet-style even k, eps 1e-3
    cases.append((2, 2, 6, 6, 7, 4, 0, "circular", 2, 1e-3))  # ConvReverseDataNet-style, per-sample psf
    cases.append((1, 2, 16, 18, 3, 3, 1, "circular", 1, 1e-5))
    cases.append((2, 2, 10, 12, 5, 1, 0, "circular", 2, 1e-3))
    arrays = {}
    for i, (B, C, H, W, k, s, p, mode, pb, eps) in enumerate(cases):
        x = rng.standard_normal((B, C, H, W)).astype(np.float32)
        w = softmax_psf(rng, pb, C, k)
        b = (0.5 * rng.standard_normal((1, C, 1, 1))).astype(np.float32)
        arrays[f"c{i}_x"] = x
        arrays[f"c{i}_w"] = w
        arrays[f"c{i}_b"] = b
        arrays[f"c{i}_meta"] = np.array([B, C, H, W, k, s, p, ["constant", "reflect", "replicate", "circular"].index(mode),
                                         pb], dtype=np.int64)
        arrays[f"c{i}_eps"] = np.array(eps, dtype=np.float64)
        arrays[f"c{i}_out64"] = module_forward(x, w, b, s, p, mode, eps, torch.float64)
        arrays[f"c{i}_out32"] = module_forward(x, w, b, s, p, mode, eps, torch.float32)
    # op level, arbitrary x0 (converse2d.cpp:165-209)
    for j, s in enumerate([1, 2, 3]):
        x = rng.standard_normal((1, 2, 10, 12)).astype(np.float32)
        x0 = rng.standard_normal((1, 2, 10 * s, 12 * s)).astype(np.float32)
        w = softmax_psf(rng, 1, 2, 3)
        b = (0.5 * rng.standard_normal((1, 2, 1, 1))).astype(np.float32)
        t = lambda a: torch.from_numpy(a).double()
        arrays[f"op{j}_x"], arrays[f"op{j}_x0"], arrays[f"op{j}_w"], arrays[f"op{j}_b"] = x, x0, w, b
        arrays[f"op{j}_s"] = np.array(s)
        arrays[f"op{j}_out64"] = torch.ops.converse2d.forward(t(x), t(x0), t(w), t(b), s, 1e-5).numpy()
    arrays["ncases"] = np.array(len(cases))
    arrays["nops"] = np.array(3)
    np.savez_compressed(os.path.join(HERE, "converse2d_ref.npz"), **arrays)
    print("wrote", len(cases), "module cases and 3 op cases")


if __name__ == "__main__":
    main()
