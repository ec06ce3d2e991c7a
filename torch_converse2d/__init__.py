"""Package name of the reference extension (Converse2D/torch_converse2d): importing it registers
torch.ops.converse2d.{forward, clear_cache} backed by the conversenet_amd HIP library, which is what
the reference's models/util_converse.py probes for (util_converse.py:15-28)."""
import conversenet_amd  # noqa: F401

__all__ = ["conversenet_amd"]
