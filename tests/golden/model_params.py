"""Seeded parameter values for the model-composition fixtures (models_ref.npz).

A fixture stores, per model, the list of (state-dict key, shape, kind) triples and one seed instead of
the parameter values (Converse-DnCNN alone has 796,353).  `seeded_state_dict` turns that list back
into the same float32 arrays on every machine: parameters are drawn one after another in list order
from numpy's PCG64 generator, each kind from its own distribution:

  psf    Converse2D.weight: softmax over the k*k taps of N(0,1), as Converse2D initialises it
  lam    Converse2D.bias (lambda = sigmoid(bias - 9) + eps): U(-1, 3)
  alpha  ConverseBlockAlphaVariant.alpha1/alpha2, ConvReverseDataNet.alpha: N(0, 0.1^2)
  ln_w   LayerNorm.weight: 1 + N(0, 0.1^2)          ln_b   LayerNorm.bias: N(0, 0.1^2)
  w      nn.Conv2d / nn.Linear weight: U(-1/sqrt(fan_in), 1/sqrt(fan_in)), fan_in = prod(shape[1:])
  b      nn.Conv2d / nn.Linear bias: U(-0.1, 0.1)

Non-zero alphas keep every residual branch visible to the comparison (they initialise to zero).
"""
import numpy as np


def _draw(rng, kind, shape):
    n = int(np.prod(shape))
    if kind == "psf":
        taps = shape[-1] * shape[-2]
        w = rng.standard_normal((n // taps, taps))
        w = np.exp(w - w.max(-1, keepdims=True))
        return (w / w.sum(-1, keepdims=True)).reshape(shape)
    if kind == "lam":
        return rng.uniform(-1.0, 3.0, shape)
    if kind == "alpha":
        return 0.1 * rng.standard_normal(shape)
    if kind == "ln_w":
        return 1.0 + 0.1 * rng.standard_normal(shape)
    if kind == "ln_b":
        return 0.1 * rng.standard_normal(shape)
    if kind == "w":
        bound = 1.0 / np.sqrt(np.prod(shape[1:]))
        return rng.uniform(-bound, bound, shape)
    if kind == "b":
        return rng.uniform(-0.1, 0.1, shape)
    raise ValueError(kind)


def seeded_state_dict(spec, seed):
    """spec: iterable of (key, shape, kind).  Returns {key: float32 ndarray}."""
    rng = np.random.default_rng(seed)
    return {key: _draw(rng, kind, tuple(shape)).astype(np.float32) for key, shape, kind in spec}
