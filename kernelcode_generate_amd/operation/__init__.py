"""DSL operations (the reference's kernel_gen.operation): `arch`, `dma`, `kernel`, `nn`, `scf`."""

from . import arch, dma, kernel, nn, scf

__all__ = ["arch", "dma", "kernel", "nn", "scf"]
