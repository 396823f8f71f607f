"""DSL operations (the reference's kernel_gen.operation): `kernel`, `dma`, `nn`, `scf`."""

from . import dma, kernel, nn, scf

__all__ = ["dma", "kernel", "nn", "scf"]
