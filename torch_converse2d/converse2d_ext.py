"""Module name the reference's extension probe tries first under this package
(models/util_converse.py:15-19: "converse2d_ext", "torch_converse2d.converse2d_ext",
"torch_converse2d").  Importing it registers torch.ops.converse2d.{forward, clear_cache,
forward_fused} backed by the conversenet_amd HIP library."""
import conversenet_amd  # noqa: F401
