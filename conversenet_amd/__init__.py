"""conversenet_amd: MI355X (gfx950) HIP implementation of ConverseNet's Converse2D forward path.

Importing the package registers torch.ops.converse2d (the reference's op namespace).  The models
and blocks live in conversenet_amd.util_converse / converse_dncnn / converse_usrnet, mirroring the
reference's models/ package.
"""
from . import _lib  # noqa: F401
from . import op_registry  # noqa: F401

__version__ = "0.1.0"
