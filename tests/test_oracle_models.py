"""Pins the oracle's model compositions against the reference's own model classes.

tests/golden/models_ref.npz holds outputs of the reference's ConverseBlock(AlphaVariant),
ConverseDnCNN, ConvReverseDataNet, KernelNet, ConverseNet, ConverseUSRNet and the Converse SRResNet
variants (models/util_converse.py:253-323, models/converse_dncnn.py:11-35,
models/converse_usrnet.py:33-214, models/converse_srresnet.py:50-119) on small seeded inputs, written
by tests/golden/make_model_golden.py in the build container.  Each case is re-run through the numpy
oracle in float64 with the same regenerated state dict.

Tolerances: float64 fixtures agree to 1e-9 relative (two FFT implementations in float64); the two
float32 fixtures (KernelNet and ConverseUSRNet run in float32 in the reference because KernelNet casts
its input to float, converse_usrnet.py:134) are compared by PSNR against the reference output, with the
thresholds below set between the float32 rounding of the reference (measured: KernelNet 161.6 dB,
USRNet 107.3 / 105.5 dB) and the planted mistakes at the end of this file (the closest: the tanh
approximation of GELU in USRNet, 93.3 dB; every wiring mistake is below 25 dB).
"""
import inspect
import json
import os
import sys

import numpy as np
import pytest

from oracle import converse_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
if os.path.join(HERE, "golden") not in sys.path:
    sys.path.insert(0, os.path.join(HERE, "golden"))
from model_params import seeded_state_dict  # noqa: E402

GOLD = np.load(os.path.join(HERE, "golden", "models_ref.npz"))
INDEX = json.loads(str(GOLD["index"]))

PSNR_FP32 = {"kernelnet": 140.0, "usrnet0": 100.0, "usrnet1": 100.0}


def case(name):
    spec = json.loads(str(GOLD[f"{name}/spec"]))
    sd = seeded_state_dict(spec, int(GOLD[f"{name}/seed"]))
    meta = json.loads(str(GOLD[f"{name}/meta"]))
    ins = [GOLD[f"{name}/in{i}"] for i in range(4) if f"{name}/in{i}" in GOLD.files]
    return sd, meta, ins, GOLD[f"{name}/out"]


def run_oracle(name, sd, meta, ins):
    if name.startswith("block"):
        return O.converse_block(ins[0], sd, "", meta["kernel_size"], 1, meta["padding"], meta["padding_mode"], 1e-5,
                                meta["alpha"])
    if name == "dncnn":
        return O.converse_dncnn(ins[0], sd)
    if name.startswith("datanet"):
        return O.conv_reverse_datanet(ins[0], ins[1], meta["sf"], sd["alpha"], 1e-3, meta["padding"],
                                      meta["padding_mode"])
    if name == "kernelnet":
        return O.kernelnet(ins[0], sd, "", 7)
    if name == "conversenet":
        return O.converse_net(ins[0], sd, meta["num_iterations"], meta["num_blocks"])
    if name.startswith("usrnet"):
        return O.converse_usrnet(ins[0], ins[1], meta["sf"], sd, 7)
    if name == "converse_msrresnet":
        return O.converse_msrresnet(ins[0], sd, meta["num_blocks"])
    if name == "converse_up_msrresnet":
        return O.converse_up_msrresnet(ins[0], sd, meta["num_blocks"])
    raise KeyError(name)


def psnr(a, ref):
    peak = float(ref.max() - ref.min())
    mse = float(np.mean((np.asarray(a, np.float64) - ref) ** 2))
    return np.inf if mse == 0 else 20 * np.log10(peak / np.sqrt(mse))


def agrees(name, got, ref):
    """(ok, figure): float64 cases by relative max-abs, float32 cases by PSNR."""
    if got.shape != ref.shape:
        return False, np.nan
    if name in PSNR_FP32:
        p = psnr(got, ref.astype(np.float64))
        return p >= PSNR_FP32[name], p
    err = float(np.abs(got - ref).max()) / max(1.0, float(np.abs(ref).max()))
    return err <= 1e-9, err


def test_fixture_covers_every_composition():
    kinds = {n.rstrip("0123456789") for n in INDEX}
    assert kinds == {"block", "dncnn", "datanet", "kernelnet", "conversenet", "usrnet", "converse_msrresnet",
                     "converse_up_msrresnet"}
    assert sum(n.startswith("block") for n in INDEX) == 5
    # non-zero alphas, so every residual branch is visible to the comparison
    sd, _, _, _ = case("usrnet0")
    assert all(np.abs(v).max() > 0 for k, v in sd.items() if "alpha" in k)


@pytest.mark.parametrize("name", INDEX)
def test_oracle_matches_reference_model(name):
    sd, meta, ins, ref = case(name)
    got = run_oracle(name, sd, meta, ins)
    ok, fig = agrees(name, got, ref)
    print(f"{name}: {'PSNR %.1f dB' % fig if name in PSNR_FP32 else 'rel max-abs %.2e' % fig}")
    assert ok, (name, fig)


# Planted mistakes, each a plausible wiring error in one composition: every one must fail its fixture.
def _mut_block_alpha(name, sd, meta, ins):
    return O.converse_block(ins[0], sd, "", meta["kernel_size"], 1, meta["padding"], meta["padding_mode"], 1e-5,
                            not meta["alpha"])


def _mut_block_ln_eps(name, sd, meta, ins, monkeypatch):
    ln = O.layernorm_cf
    monkeypatch.setattr(O, "layernorm_cf", lambda x, w, b, eps, dtype=np.float64: ln(x, w, b, 1e-6, dtype))
    return run_oracle(name, sd, meta, ins)


def _mut_gelu_tanh(name, sd, meta, ins, monkeypatch):
    monkeypatch.setattr(O, "gelu", lambda x: 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3))))
    return run_oracle(name, sd, meta, ins)


def _mut_kernelnet_no_gelu2(name, sd, meta, ins, monkeypatch):
    calls = []
    gelu = O.gelu

    def g(x):
        calls.append(1)
        return x if len(calls) == 2 else gelu(x)

    monkeypatch.setattr(O, "gelu", g)
    return run_oracle(name, sd, meta, ins)


def _mut_dncnn_19(name, sd, meta, ins):
    return O.converse_dncnn(ins[0], sd, num_blocks=19)


def _mut_datanet_zero_x0(name, sd, meta, ins, monkeypatch):
    monkeypatch.setattr(O, "nearest", lambda x, s: O.upsample_zero(x, s))
    return run_oracle(name, sd, meta, ins)


def _mut_datanet_eps(name, sd, meta, ins):
    return O.conv_reverse_datanet(ins[0], ins[1], meta["sf"], sd["alpha"], 1e-5, meta["padding"], meta["padding_mode"])


def _mut_usrnet_convs0(name, sd, meta, ins):
    sd = dict(sd)
    for i in range(1, 5):
        sd[f"convs.{i}.weight"], sd[f"convs.{i}.bias"] = sd["convs.0.weight"], sd["convs.0.bias"]
    return run_oracle(name, sd, meta, ins)


def _mut_conversenet_iters(name, sd, meta, ins):
    return O.converse_net(ins[0], sd, meta["num_iterations"] - 1, meta["num_blocks"])


MUTANTS = [("block1", _mut_block_alpha), ("block4", _mut_block_alpha), ("block3", _mut_block_ln_eps),
           ("block2", _mut_gelu_tanh), ("dncnn", _mut_dncnn_19), ("datanet2", _mut_datanet_zero_x0),
           ("datanet3", _mut_datanet_zero_x0), ("datanet0", _mut_datanet_eps), ("kernelnet", _mut_kernelnet_no_gelu2),
           ("usrnet0", _mut_usrnet_convs0), ("usrnet1", _mut_gelu_tanh), ("conversenet", _mut_conversenet_iters),
           ("converse_msrresnet", _mut_gelu_tanh)]


@pytest.mark.parametrize("name,mut", MUTANTS, ids=[f"{n}-{m.__name__}" for n, m in MUTANTS])
def test_planted_mistake_fails_fixture(name, mut, monkeypatch):
    sd, meta, ins, ref = case(name)
    args = (name, sd, meta, ins, monkeypatch) if "monkeypatch" in inspect.signature(mut).parameters else (
        name, sd, meta, ins)
    ok, fig = agrees(name, mut(*args), ref)
    print(f"{name} {mut.__name__}: {fig}")
    assert not ok, (name, mut.__name__, fig)
