"""Registers the reference's operator namespace `converse2d` backed by the HIP library.

Schema kept identical to Converse2D/torch_converse2d/converse2d.cpp:218-222:
    converse2d::forward(Tensor x, Tensor x0, Tensor weight, Tensor bias, int scale, float eps=1e-5)
    converse2d::clear_cache() -> ()
plus the module-level fused entry point used by conversenet_amd.util_converse.Converse2D:
    converse2d::forward_fused(Tensor x, Tensor weight, Tensor bias, int scale, int padding,
                              str padding_mode, float eps=1e-5, str act="none") -> Tensor

Like the reference (CompositeImplicitAutograd, converse2d.cpp:223-227) the kernels are registered
for every backend: fp32 HIP tensors that need no gradient run the HIP library; everything else
(CPU tensors, other dtypes, grad-requiring inputs) runs the torch.fft composition, which autograd
differentiates.  Importing this module is what makes `torch.ops.converse2d.forward` exist, which is
how the reference's models/util_converse.py discovers an extension (:10-34).
"""
from __future__ import annotations

import torch

from . import _lib, composite, functional

_LIB = None


def _hip_ok(*ts) -> bool:
    if not all(t.is_cuda and t.dtype == torch.float32 for t in ts):
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
        return False
    _lib.load()  # HIP tensors need the library: ImportError rather than a silent fallback
    return True


def _forward(x, x0, weight, bias, scale, eps=1e-5):
    # geometries past the library's limits (e.g. a padded side above 4096, too many planes for the
    # multi-pass grid) run the composition, which has none, instead of raising CVN_ERR_UNSUPPORTED
    if _hip_ok(x, x0, weight, bias) and functional.op_supported(x, x0, weight, scale):
        return functional.converse2d_op(x, x0, weight, bias, scale, eps)
    return composite.converse2d_op(x, x0, weight, bias, scale, eps)


def _forward_fused(x, weight, bias, scale, padding, padding_mode, eps=1e-5, act="none"):
    if _hip_ok(x, weight, bias) and functional.supported(x, weight, scale, padding):
        return functional.converse2d_fused(x, weight, bias.reshape(-1), scale, padding, padding_mode, eps,
                                           act if act != "none" else None)
    out = composite.converse2d_module(x, weight, bias.reshape(1, -1, 1, 1), scale, padding, padding_mode, eps)
    if act == "gelu":
        out = torch.nn.functional.gelu(out)
    return out


def _clear_cache():
    """Drops the cached transfer tables (the reference clears its OTF cache, converse2d.cpp:211-216)."""
    functional.table_cache.clear()
    functional.release_workspace()


def register():
    """Define the namespace once per process (raises if another library already owns it)."""
    global _LIB
    if _LIB is not None:
        return
    lib = torch.library.Library("converse2d", "DEF")
    lib.define("forward(Tensor x, Tensor x0, Tensor weight, Tensor bias, int scale, float eps=1e-5) -> Tensor")
    lib.define("clear_cache() -> ()")
    lib.define("forward_fused(Tensor x, Tensor weight, Tensor bias, int scale, int padding, str padding_mode, "
               "float eps=1e-5, str act=\"none\") -> Tensor")
    lib.impl("forward", _forward, "CompositeImplicitAutograd")
    lib.impl("forward_fused", _forward_fused, "CompositeImplicitAutograd")
    lib.impl("clear_cache", _clear_cache, "CompositeImplicitAutograd")
    _LIB = lib


register()
