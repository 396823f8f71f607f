"""IR passes of the gfx950 lowering pipeline: kernel-aggregate (aggregate.py) and
kernel-pattern-fuse (fuse.py)."""

from .aggregate import kernel_aggregate
from .fuse import FusedCall, pattern_fuse

__all__ = ["FusedCall", "kernel_aggregate", "pattern_fuse"]
